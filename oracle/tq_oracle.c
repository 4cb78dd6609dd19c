/*
 * tq_oracle.c — CPU oracle (test infrastructure only; see tq_oracle.h).
 *
 * Build: gcc -O2 -std=c99 -ffp-contract=off -fPIC -shared (oracle/build_oracle.sh).
 * No -ffast-math: every float operation below is one IEEE binary32 RNE
 * operation in the order the reference's device code performs it.
 */
#define _GNU_SOURCE
#include "tq_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define TQO_MAX_D 128

/* Codebook literals: src/cuda/tq_turbo_prod_kernels.cu:26-37 (K3, V4) and
 * src/cuda/tq_turbo_mse_kernels.cu:24-29 (the turbo_mse table equals V4). */
static const float kK3[8] = {-2.1513f, -1.34326f, -0.755526f, -0.244919f,
                             0.244919f, 0.755526f, 1.34326f,  2.1513f};
static const float kV4[16] = {-2.7326f, -2.0690f, -1.6180f, -1.2562f, -0.9423f, -0.6568f,
                              -0.3880f, -0.1284f, 0.1284f,  0.3880f,  0.6568f,  0.9423f,
                              1.2562f,  1.6180f,  2.0690f,  2.7326f};

float tqo_k3(int i) { return kK3[i & 7]; }
float tqo_v4(int i) { return kV4[i & 15]; }

/* ------------------------------------------------------------------------ */
/* binary16 conversions                                                      */
/* ------------------------------------------------------------------------ */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Round m right by s bits, to nearest, ties to even. */
static uint64_t rne_shift(uint64_t m, int s) {
    if (s <= 0) return m;
    if (s >= 64) return 0;
    uint64_t q = m >> s;
    uint64_t r = m & ((1ull << s) - 1);
    uint64_t half = 1ull << (s - 1);
    if (r > half || (r == half && (q & 1))) q++;
    return q;
}

uint16_t tqo_f2h(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7fffffffu;
    uint32_t e = a >> 23, m = a & 0x7fffffu;
    if (e == 0xff) return (uint16_t)(sign | (m ? (0x7e00u | (m >> 13)) : 0x7c00u));
    if (e >= 143) return (uint16_t)(sign | 0x7c00u); /* >= 2^16 */
    if (e >= 113) {                                   /* fp16-normal range */
        uint64_t comb = ((uint64_t)(e - 112) << 23) | m;
        uint64_t h = rne_shift(comb, 13);             /* carry may reach inf */
        if (h >= 0x7c00u) h = 0x7c00u;
        return (uint16_t)(sign | h);
    }
    /* fp16 subnormal or zero: value / 2^-24 = mant * 2^(e - 126) */
    if (e == 0) return sign; /* fp32 subnormal: < 2^-126, rounds to 0 */
    uint64_t mant = (uint64_t)m | 0x800000u;
    int shift = 126 - (int)e; /* >= 14 */
    return (uint16_t)(sign | rne_shift(mant, shift));
}

float tqo_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        float v = (float)m * 0x1p-24f; /* exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112) << 23) | (m << 13));
}

void tqo_f2h_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = tqo_f2h(in[i]);
}
void tqo_h2f_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = tqo_h2f(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Rotation, codebooks, reductions                                           */
/* ------------------------------------------------------------------------ */

/* rsqrtf((float)D) at :188/:336; this build uses the correctly rounded value
 * RN(2^(-k/2)): exact for even k, RN(1/sqrt(2)) * 2^-((k-1)/2) for odd k. */
float tqo_inv_sqrt_d(int D) {
    int k = 0;
    while ((1 << k) < D) ++k;
    if ((k & 1) == 0) return ldexpf(1.0f, -k / 2);
    return ldexpf(0x1.6a09e6p-1f, -(k - 1) / 2);
}

/* src/cuda/tq_turbo_prod_kernels.cu:19-23 (identical in turbo_mse :18-22). */
float tqo_sign_flip(int idx, int head) {
    unsigned x = ((unsigned)head * 2654435761u) ^ ((unsigned)idx * 1103515245u + 12345u);
    return (x & 1u) ? 1.0f : -1.0f;
}

static float clampf_ref(float x, float lo, float hi) { /* clamp_val, :14-17 */
    return x < lo ? lo : (x > hi ? hi : x);
}

/* nearest_k3_idx / nearest_v4_idx, :39-59: strict '<' keeps the first min. */
int tqo_nearest_k3(float x) {
    int best = 0;
    float bd = fabsf(x - kK3[0]);
    for (int i = 1; i < 8; ++i) {
        float d = fabsf(x - kK3[i]);
        if (d < bd) { bd = d; best = i; }
    }
    return best;
}

int tqo_nearest_v4(float x) {
    int best = 0;
    float bd = fabsf(x - kV4[0]);
    for (int i = 1; i < 16; ++i) {
        float d = fabsf(x - kV4[i]);
        if (d < bd) { bd = d; best = i; }
    }
    return best;
}

/* hadamard_inplace, :89-105: unnormalised, stages len = 1, 2, ..., D/2. */
void tqo_wht(float* x, int D) {
    for (int len = 1; len < D; len <<= 1) {
        for (int t = 0; t < (D >> 1); ++t) {
            int group = t / len, offset = t % len;
            int i0 = group * (len << 1) + offset, i1 = i0 + len;
            float a = x[i0], b = x[i1];
            x[i0] = a + b;
            x[i1] = a - b;
        }
    }
}

static void wht_f64(double* x, int D) {
    for (int len = 1; len < D; len <<= 1)
        for (int t = 0; t < (D >> 1); ++t) {
            int i0 = (t / len) * (len << 1) + t % len, i1 = i0 + len;
            double a = x[i0], b = x[i1];
            x[i0] = a + b;
            x[i1] = a - b;
        }
}

/* The shared-memory tree of :195-198: r[i] += r[i + stride], stride halving. */
float tqo_tree_sum(const float* r_in, int n) {
    float r[TQO_MAX_D];
    memcpy(r, r_in, sizeof(float) * (size_t)n);
    for (int s = n >> 1; s > 0; s >>= 1)
        for (int i = 0; i < s; ++i) r[i] += r[i + s];
    return r[0];
}

static float rms_of(const float* red, int n, int D) {
    float v = sqrtf(tqo_tree_sum(red, n) / (float)D);
    if (v < 1e-8f) v = 1e-8f; /* kMinRMS, include/tq_shared_device.cuh:9 */
    return v;
}

static void put_h(uint8_t* p, uint16_t h) { p[0] = (uint8_t)(h & 0xff); p[1] = (uint8_t)(h >> 8); }
static uint16_t get_h(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static int nib_get(const uint8_t* src, int i) { /* unpack_4bit_get, tq_shared_device.cuh:61-64 */
    uint8_t b = src[i >> 1];
    return (i & 1) ? (b >> 4) & 0xf : b & 0xf;
}

/* ------------------------------------------------------------------------ */
/* Layouts                                                                   */
/* ------------------------------------------------------------------------ */

static size_t align_up(size_t x, size_t a) { return ((x + a - 1) / a) * a; }

/* src/tq_turbo_prod.cpp:7-39 */
void tqo_make_prod_layout(int block_size, int H, int D, tqo_prod_layout* L) {
    memset(L, 0, sizeof(*L));
    L->k4_bytes = (D + 1) / 2;
    L->v4_bytes = (D * 4 + 7) / 8;
    L->scale_bytes = 2;
    size_t th = (size_t)block_size * (size_t)H, cur = 0;
    L->k4_off = cur; cur += th * (size_t)L->k4_bytes;
    cur = align_up(cur, 2);
    L->kres_off = cur; cur += th * 2;
    L->ks_off = cur; cur += th * 2;
    L->v4_off = cur; cur += th * (size_t)L->v4_bytes;
    cur = align_up(cur, 2);
    L->vs_off = cur; cur += th * 2;
    L->page_size = align_up(cur, 2);
}

/* src/tq_turbo_mse_layout.cpp:7-28 */
void tqo_make_mse_layout(int block_size, int H, int D, int nbits, int page_alignment,
                         tqo_mse_layout* L) {
    memset(L, 0, sizeof(*L));
    L->code_bytes = (size_t)((D * nbits + 7) / 8);
    L->norm_bytes = 2;
    size_t th = (size_t)block_size * (size_t)H, a = (size_t)page_alignment;
    L->k_codes_off = 0;
    L->v_codes_off = align_up(L->k_codes_off + th * L->code_bytes, a);
    L->k_norms_off = align_up(L->v_codes_off + th * L->code_bytes, a);
    L->v_norms_off = align_up(L->k_norms_off + th * L->norm_bytes, a);
    L->page_size = align_up(L->v_norms_off + th * L->norm_bytes, a);
}

/* ------------------------------------------------------------------------ */
/* Thread pool helper                                                        */
/* ------------------------------------------------------------------------ */

typedef void (*row_fn)(void* ctx, long long row);
typedef struct { row_fn fn; void* ctx; long long begin, end; } span_t;

static void* span_run(void* p) {
    span_t* s = (span_t*)p;
    for (long long r = s->begin; r < s->end; ++r) s->fn(s->ctx, r);
    return NULL;
}

static void parallel_rows(long long n, int nthreads, row_fn fn, void* ctx) {
    if (nthreads <= 1 || n < 2) {
        for (long long r = 0; r < n; ++r) fn(ctx, r);
        return;
    }
    if (nthreads > 256) nthreads = 256;
    if (nthreads > n) nthreads = (int)n;
    pthread_t th[256];
    span_t sp[256];
    for (int i = 0; i < nthreads; ++i) {
        sp[i].fn = fn; sp[i].ctx = ctx;
        sp[i].begin = n * i / nthreads;
        sp[i].end = n * (i + 1) / nthreads;
        pthread_create(&th[i], NULL, span_run, &sp[i]);
    }
    for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------ */
/* turbo_prod pack / dequant                                                 */
/* ------------------------------------------------------------------------ */

/* Rotation of one token-head: x_i = f32(src_i) * s_i; WHT; x_i *= inv
 * (:181-190, turbo_mse :78-107). */
static void rotate_row(const uint16_t* src, int head, int D, float* x) {
    float inv = tqo_inv_sqrt_d(D);
    for (int i = 0; i < D; ++i) x[i] = tqo_h2f(src[i]) * tqo_sign_flip(i, head);
    tqo_wht(x, D);
    for (int i = 0; i < D; ++i) x[i] *= inv;
}

/* B.1: src/cuda/tq_turbo_prod_kernels.cu:180-259 for one (token, head).
 * The optional outputs are the reference kernel's debug buffers
 * (:216-217, :243-246): rotated K/V, clamped normalised K/V, code indices. */
void tqo_prod_pack_row_debug(const uint16_t* k, const uint16_t* v, int head, int D, uint8_t* k4,
                             uint8_t* v4, uint16_t* ks, uint16_t* kres, uint16_t* vs,
                             float* krot_out, float* vrot_out, float* kn_out, float* vn_out,
                             int* kidx_out, int* vidx_out) {
    float sk[TQO_MAX_D], sv[TQO_MAX_D], red[TQO_MAX_D], e[TQO_MAX_D];
    int kc[TQO_MAX_D], kb[TQO_MAX_D], vc[TQO_MAX_D];
    rotate_row(k, head, D, sk);
    rotate_row(v, head, D, sv);
    for (int i = 0; i < D; ++i) {
        if (krot_out) krot_out[i] = sk[i];
        if (vrot_out) vrot_out[i] = sv[i];
    }
    for (int i = 0; i < D; ++i) red[i] = sk[i] * sk[i];
    float krms = rms_of(red, D, D);
    *ks = tqo_f2h(krms);
    for (int i = 0; i < D; ++i) red[i] = sv[i] * sv[i];
    float vrms = rms_of(red, D, D);
    *vs = tqo_f2h(vrms);
    for (int i = 0; i < D; ++i) {
        float kn = clampf_ref(sk[i] / krms, -2.5f, 2.5f);
        float vn = clampf_ref(sv[i] / vrms, -2.75f, 2.75f);
        if (kn_out) kn_out[i] = kn;
        if (vn_out) vn_out[i] = vn;
        kc[i] = tqo_nearest_k3(kn);
        e[i] = kn - kK3[kc[i]];
        kb[i] = (e[i] >= 0.0f) ? 1 : 0;
        vc[i] = tqo_nearest_v4(vn);
        if (kidx_out) kidx_out[i] = kc[i];
        if (vidx_out) vidx_out[i] = vc[i];
    }
    for (int i = 0; i < D; ++i) red[i] = e[i] * e[i];
    *kres = tqo_f2h(rms_of(red, D, D));
    for (int j = 0; j < D / 2; ++j) {
        int a = (kb[2 * j] << 3) | kc[2 * j], b = (kb[2 * j + 1] << 3) | kc[2 * j + 1];
        k4[j] = (uint8_t)(a | (b << 4));
        v4[j] = (uint8_t)(vc[2 * j] | (vc[2 * j + 1] << 4));
    }
}

void tqo_prod_pack_row(const uint16_t* k, const uint16_t* v, int head, int D, uint8_t* k4,
                       uint8_t* v4, uint16_t* ks, uint16_t* kres, uint16_t* vs, float* kn_out,
                       float* vn_out) {
    tqo_prod_pack_row_debug(k, v, head, D, k4, v4, ks, kres, vs, NULL, NULL, kn_out, vn_out, NULL,
                            NULL);
}

typedef struct {
    const uint16_t *key, *value;
    int H, D;
    float *krot, *vrot, *kn, *vn;
    int *kidx, *vidx;
} dbg_ctx;

static void prod_debug_one(void* p, long long row) {
    dbg_ctx* c = (dbg_ctx*)p;
    const size_t off = (size_t)row * (size_t)c->D;
    uint8_t k4[TQO_MAX_D / 2], v4[TQO_MAX_D / 2];
    uint16_t a, b, cc;
#define TQO_AT(ptr) ((ptr) ? (ptr) + off : NULL)
    tqo_prod_pack_row_debug(c->key + off, c->value + off, (int)(row % c->H), c->D, k4, v4, &a, &b,
                            &cc, TQO_AT(c->krot), TQO_AT(c->vrot), TQO_AT(c->kn), TQO_AT(c->vn),
                            TQO_AT(c->kidx), TQO_AT(c->vidx));
#undef TQO_AT
}

void tqo_prod_pack_debug(const uint16_t* key, const uint16_t* value, int num_tokens, int H, int D,
                         float* krot, float* vrot, float* kn, float* vn, int* kidx, int* vidx,
                         int nthreads) {
    dbg_ctx c = {key, value, H, D, krot, vrot, kn, vn, kidx, vidx};
    parallel_rows((long long)num_tokens * H, nthreads, prod_debug_one, &c);
}

typedef struct {
    const uint16_t *key, *value;
    const int32_t* slots;
    const uint8_t* cpool;
    uint8_t* pool;
    uint16_t *ok, *ov;
    int H, D, bs, fused;
    const tqo_prod_layout* PL;
    const tqo_mse_layout* ML;
} kv_ctx;

static void prod_pack_one(void* p, long long row) {
    kv_ctx* c = (kv_ctx*)p;
    int t = (int)(row / c->H), h = (int)(row % c->H);
    int slot = c->slots[t];
    if (slot < 0) return;
    int page = slot / c->bs, tib = slot % c->bs, cell = tib * c->H + h;
    uint8_t* base = c->pool + (size_t)page * c->PL->page_size;
    uint16_t ks, kres, vs;
    const size_t off = (size_t)row * (size_t)c->D;
    tqo_prod_pack_row(c->key + off, c->value + off, h, c->D,
                      base + c->PL->k4_off + (size_t)cell * (size_t)c->PL->k4_bytes,
                      base + c->PL->v4_off + (size_t)cell * (size_t)c->PL->v4_bytes, &ks, &kres,
                      &vs, NULL, NULL);
    put_h(base + c->PL->ks_off + (size_t)cell * 2, ks);
    put_h(base + c->PL->kres_off + (size_t)cell * 2, kres);
    put_h(base + c->PL->vs_off + (size_t)cell * 2, vs);
}

void tqo_prod_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                   int num_tokens, int H, int D, int block_size, const tqo_prod_layout* L,
                   uint8_t* pool, int nthreads) {
    kv_ctx c = {key, value, slots, NULL, pool, NULL, NULL, H, D, block_size, 0, L, NULL};
    parallel_rows((long long)num_tokens * H, nthreads, prod_pack_one, &c);
}

/* B.3: src/cuda/tq_turbo_prod_kernels.cu:315-340. */
static void prod_dequant_one(void* p, long long row) {
    kv_ctx* c = (kv_ctx*)p;
    int t = (int)(row / c->H), h = (int)(row % c->H), D = c->D;
    int slot = c->slots[t];
    if (slot < 0) return;
    int page = slot / c->bs, tib = slot % c->bs, cell = tib * c->H + h;
    const uint8_t* base = c->cpool + (size_t)page * c->PL->page_size;
    const uint8_t* k4 = base + c->PL->k4_off + (size_t)cell * (size_t)c->PL->k4_bytes;
    const uint8_t* v4 = base + c->PL->v4_off + (size_t)cell * (size_t)c->PL->v4_bytes;
    float ks = tqo_h2f(get_h(base + c->PL->ks_off + (size_t)cell * 2));
    float re = tqo_h2f(get_h(base + c->PL->kres_off + (size_t)cell * 2));
    float vs = tqo_h2f(get_h(base + c->PL->vs_off + (size_t)cell * 2));
    float sk[TQO_MAX_D], sv[TQO_MAX_D];
    for (int i = 0; i < D; ++i) {
        int nib = nib_get(k4, i);
        float sign_e = ((nib >> 3) & 1) ? 1.0f : -1.0f;
        float kval = kK3[nib & 7] + re * sign_e;
        sk[i] = kval * ks;
        sv[i] = kV4[nib_get(v4, i)] * vs;
    }
    tqo_wht(sk, D);
    tqo_wht(sv, D);
    float inv = tqo_inv_sqrt_d(D);
    const size_t off = (size_t)row * (size_t)D;
    for (int i = 0; i < D; ++i) {
        float s = tqo_sign_flip(i, h);
        c->ok[off + i] = tqo_f2h(sk[i] * inv * s);
        c->ov[off + i] = tqo_f2h(sv[i] * inv * s);
    }
}

void tqo_prod_dequant(const uint8_t* pool, const int32_t* slots, int num_tokens, int H, int D,
                      int block_size, const tqo_prod_layout* L, uint16_t* out_key,
                      uint16_t* out_value, int nthreads) {
    kv_ctx c = {NULL, NULL, slots, pool, NULL, out_key, out_value, H, D, block_size, 0, L, NULL};
    parallel_rows((long long)num_tokens * H, nthreads, prod_dequant_one, &c);
}

/* ------------------------------------------------------------------------ */
/* turbo_prod attention                                                      */
/* ------------------------------------------------------------------------ */

typedef struct {
    const uint16_t* q;
    const uint8_t* pool;
    const int32_t* slots;
    int Q, N, H, D, bs;
    const tqo_prod_layout* PL;
    const tqo_mse_layout* ML;
    float* logits_f;
    double* out_d;
    double* logits_d;
    uint16_t* out_h;
} att_ctx;

typedef struct {
    const uint8_t* k;  /* K codes of the cell */
    const uint8_t* v;  /* V codes of the cell */
    float ks, re, vs;
} cell_t;

static void prod_cell(const att_ctx* c, int t, int h, cell_t* out) {
    int slot = c->slots[t];
    int page = slot / c->bs, tib = slot % c->bs, cell = tib * c->H + h;
    const uint8_t* base = c->pool + (size_t)page * c->PL->page_size;
    out->k = base + c->PL->k4_off + (size_t)cell * (size_t)c->PL->k4_bytes;
    out->v = base + c->PL->v4_off + (size_t)cell * (size_t)c->PL->v4_bytes;
    out->ks = tqo_h2f(get_h(base + c->PL->ks_off + (size_t)cell * 2));
    out->re = tqo_h2f(get_h(base + c->PL->kres_off + (size_t)cell * 2));
    out->vs = tqo_h2f(get_h(base + c->PL->vs_off + (size_t)cell * 2));
}

static void mse_cell(const att_ctx* c, int t, int h, cell_t* out) {
    int slot = c->slots[t];
    int page = slot / c->bs, tib = slot % c->bs, cell = tib * c->H + h;
    const uint8_t* base = c->pool + (size_t)page * c->ML->page_size;
    out->k = base + c->ML->k_codes_off + (size_t)cell * c->ML->code_bytes;
    out->v = base + c->ML->v_codes_off + (size_t)cell * c->ML->code_bytes;
    out->ks = tqo_h2f(get_h(base + c->ML->k_norms_off + (size_t)cell * c->ML->norm_bytes));
    out->re = 0.0f;
    out->vs = tqo_h2f(get_h(base + c->ML->v_norms_off + (size_t)cell * c->ML->norm_bytes));
}

/* qrot = WHT(q * s) * inv in fp32 (:472-478). */
static void rotate_query(const att_ctx* c, int qi, int h, float* qrot) {
    rotate_row(c->q + ((size_t)qi * c->H + h) * (size_t)c->D, h, c->D, qrot);
}

/* Logits kernel, :372-431, fp32 in the reference's order. */
static void prod_logits_one(void* p, long long row) {
    att_ctx* c = (att_ctx*)p;
    int qi = (int)(row / c->H), h = (int)(row % c->H), D = c->D;
    float qrot[TQO_MAX_D], red[TQO_MAX_D];
    rotate_query(c, qi, h, qrot);
    float inv = tqo_inv_sqrt_d(D);
    for (int t = 0; t < c->N; ++t) {
        cell_t ce;
        if (c->slots[t] < 0) { /* this build's extension: unmapped token */
            c->logits_f[((size_t)qi * c->H + h) * (size_t)c->N + t] = -INFINITY;
            continue;
        }
        prod_cell(c, t, h, &ce);
        float res_ks = ce.ks * ce.re;
        for (int i = 0; i < D; ++i) red[i] = qrot[i] * kK3[nib_get(ce.k, i) & 7] * ce.ks;
        float base = tqo_tree_sum(red, D);
        for (int i = 0; i < D; ++i)
            red[i] = qrot[i] * (((nib_get(ce.k, i) >> 3) & 1) ? 1.0f : -1.0f);
        float s2 = tqo_tree_sum(red, D);
        c->logits_f[((size_t)qi * c->H + h) * (size_t)c->N + t] = (base + s2 * res_ks) * inv;
    }
}

void tqo_prod_logits_f32(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                         int num_queries, int num_kv_tokens, int H, int D, int block_size,
                         const tqo_prod_layout* L, float* logits, int nthreads) {
    att_ctx c = {query, pool, slots, num_queries, num_kv_tokens, H, D, block_size, L, NULL,
                 logits, NULL, NULL, NULL};
    parallel_rows((long long)num_queries * H, nthreads, prod_logits_one, &c);
}

/* Exact (fp64) attention over the codes.  is_prod selects the K decode:
 *   prod: logit = ks*(sum qrot*K3[c] + re*sum qrot*sign)/sqrt(D)
 *   mse : logit = ks*(sum qrot*V4[c])/sqrt(D)
 * then softmax, acc = sum p*vs*V4[v], acc /= l, inverse WHT, * s_i/sqrt(D). */
static void attention_f64_one(att_ctx* c, long long row, int is_prod) {
    int qi = (int)(row / c->H), h = (int)(row % c->H), D = c->D, N = c->N;
    float qrot[TQO_MAX_D];
    double qd[TQO_MAX_D], acc[TQO_MAX_D];
    rotate_query(c, qi, h, qrot);
    for (int i = 0; i < D; ++i) { qd[i] = (double)qrot[i]; acc[i] = 0.0; }
    double invd = 1.0 / sqrt((double)D);
    double* lg = (double*)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
    double mx = -INFINITY;
    for (int t = 0; t < N; ++t) {
        cell_t ce;
        if (c->slots[t] < 0) { lg[t] = -INFINITY; continue; } /* unmapped token */
        if (is_prod) prod_cell(c, t, h, &ce); else mse_cell(c, t, h, &ce);
        double s1 = 0.0, s2 = 0.0;
        for (int i = 0; i < D; ++i) {
            int nib = nib_get(ce.k, i);
            if (is_prod) {
                s1 += qd[i] * (double)kK3[nib & 7];
                s2 += ((nib >> 3) & 1) ? qd[i] : -qd[i];
            } else {
                s1 += qd[i] * (double)kV4[nib];
            }
        }
        lg[t] = (double)ce.ks * (s1 + (double)ce.re * s2) * invd;
        if (lg[t] > mx) mx = lg[t];
    }
    double l = 0.0;
    for (int t = 0; t < N; ++t) {
        cell_t ce;
        if (c->slots[t] < 0) continue;
        if (is_prod) prod_cell(c, t, h, &ce); else mse_cell(c, t, h, &ce);
        double w = exp(lg[t] - mx);
        l += w;
        for (int i = 0; i < D; ++i) acc[i] += w * (double)ce.vs * (double)kV4[nib_get(ce.v, i)];
    }
    if (c->logits_d)
        for (int t = 0; t < N; ++t) c->logits_d[((size_t)qi * c->H + h) * (size_t)N + t] = lg[t];
    free(lg);
    if (l > 0.0)
        for (int i = 0; i < D; ++i) acc[i] /= l;
    wht_f64(acc, D);
    double* o = c->out_d + ((size_t)qi * c->H + h) * (size_t)D;
    for (int i = 0; i < D; ++i) o[i] = acc[i] * invd * (double)tqo_sign_flip(i, h);
}

static void prod_att64_one(void* p, long long row) { attention_f64_one((att_ctx*)p, row, 1); }
static void mse_att64_one(void* p, long long row) { attention_f64_one((att_ctx*)p, row, 0); }

void tqo_prod_attention_f64(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                            int num_queries, int num_kv_tokens, int H, int D, int block_size,
                            const tqo_prod_layout* L, double* out, double* logits,
                            int nthreads) {
    att_ctx c = {query, pool, slots, num_queries, num_kv_tokens, H, D, block_size, L, NULL,
                 NULL, out, logits, NULL};
    parallel_rows((long long)num_queries * H, nthreads, prod_att64_one, &c);
}

/* The reference kernel's algorithm in fp32 (:473-570 prod, turbo_mse
 * :336-416): tree-reduced logits, thread-0 online softmax with expf from
 * m = -1e30, V accumulated in the rotated domain, 1/l, WHT, fp16. */
static void attention_f32_one(att_ctx* c, long long row, int is_prod) {
    int qi = (int)(row / c->H), h = (int)(row % c->H), D = c->D;
    float qrot[TQO_MAX_D], vacc[TQO_MAX_D], red[TQO_MAX_D];
    rotate_query(c, qi, h, qrot);
    float inv = tqo_inv_sqrt_d(D);
    for (int i = 0; i < D; ++i) vacc[i] = 0.0f;
    float m = -1e30f, l = 0.0f; /* kInitMaxLogit */
    for (int t = 0; t < c->N; ++t) {
        cell_t ce;
        float logit;
        if (c->slots[t] < 0) continue; /* unmapped token (this build's extension) */
        if (is_prod) {
            prod_cell(c, t, h, &ce);
            float res_ks = ce.ks * ce.re;
            for (int i = 0; i < D; ++i) red[i] = qrot[i] * kK3[nib_get(ce.k, i) & 7] * ce.ks;
            float base = tqo_tree_sum(red, D);
            for (int i = 0; i < D; ++i)
                red[i] = qrot[i] * (((nib_get(ce.k, i) >> 3) & 1) ? 1.0f : -1.0f);
            logit = (base + tqo_tree_sum(red, D) * res_ks) * inv;
        } else {
            mse_cell(c, t, h, &ce);
            for (int i = 0; i < D; ++i) red[i] = qrot[i] * (kV4[nib_get(ce.k, i)] * ce.ks);
            logit = tqo_tree_sum(red, D) * inv;
        }
        float m_new = fmaxf(m, logit);
        float a = expf(m - m_new), b = expf(logit - m_new);
        l = l * a + b;
        m = m_new;
        for (int i = 0; i < D; ++i) {
            vacc[i] *= a;
            vacc[i] += b * (kV4[nib_get(ce.v, i)] * ce.vs);
        }
    }
    float inv_l = (l > 0.0f) ? (1.0f / l) : 1.0f;
    for (int i = 0; i < D; ++i) vacc[i] *= inv_l;
    tqo_wht(vacc, D);
    uint16_t* o = c->out_h + ((size_t)qi * c->H + h) * (size_t)D;
    for (int i = 0; i < D; ++i) o[i] = tqo_f2h(vacc[i] * inv * tqo_sign_flip(i, h));
}

static void prod_att32_one(void* p, long long row) { attention_f32_one((att_ctx*)p, row, 1); }
static void mse_att32_one(void* p, long long row) { attention_f32_one((att_ctx*)p, row, 0); }

void tqo_prod_attention_f32(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                            int num_queries, int num_kv_tokens, int H, int D, int block_size,
                            const tqo_prod_layout* L, uint16_t* out, int nthreads) {
    att_ctx c = {query, pool, slots, num_queries, num_kv_tokens, H, D, block_size, L, NULL,
                 NULL, NULL, NULL, out};
    parallel_rows((long long)num_queries * H, nthreads, prod_att32_one, &c);
}

/* ------------------------------------------------------------------------ */
/* turbo_mse                                                                 */
/* ------------------------------------------------------------------------ */

/* B.2: cooperative_forward_transform_and_quantize, tq_turbo_mse_kernels.cu:65-136. */
void tqo_mse_pack_row(const uint16_t* src, int head, int D, int fused, uint8_t* codes,
                      uint16_t* norm, float* xn) {
    float x[TQO_MAX_D], red[TQO_MAX_D / 2];
    rotate_row(src, head, D, x);
    for (int t = 0; t < D / 2; ++t) {
        float a = x[2 * t], b = x[2 * t + 1];
        red[t] = fused ? fmaf(a, a, b * b) : a * a + b * b;
    }
    float rms = rms_of(red, D / 2, D);
    *norm = tqo_f2h(rms);
    for (int t = 0; t < D / 2; ++t) {
        float a = clampf_ref(x[2 * t] / rms, -2.75f, 2.75f);
        float b = clampf_ref(x[2 * t + 1] / rms, -2.75f, 2.75f);
        if (xn) { xn[2 * t] = a; xn[2 * t + 1] = b; }
        codes[t] = (uint8_t)((tqo_nearest_v4(b) << 4) | tqo_nearest_v4(a));
    }
}

static void mse_pack_one(void* p, long long row) {
    kv_ctx* c = (kv_ctx*)p;
    int t = (int)(row / c->H), h = (int)(row % c->H);
    int slot = c->slots[t];
    if (slot < 0) return;
    int page = slot / c->bs, tib = slot % c->bs, cell = tib * c->H + h;
    uint8_t* base = c->pool + (size_t)page * c->ML->page_size;
    const size_t off = (size_t)row * (size_t)c->D;
    uint16_t kn, vn;
    tqo_mse_pack_row(c->key + off, h, c->D, c->fused,
                     base + c->ML->k_codes_off + (size_t)cell * c->ML->code_bytes, &kn, NULL);
    tqo_mse_pack_row(c->value + off, h, c->D, c->fused,
                     base + c->ML->v_codes_off + (size_t)cell * c->ML->code_bytes, &vn, NULL);
    put_h(base + c->ML->k_norms_off + (size_t)cell * c->ML->norm_bytes, kn);
    put_h(base + c->ML->v_norms_off + (size_t)cell * c->ML->norm_bytes, vn);
}

void tqo_mse_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                  int num_tokens, int H, int D, int block_size, const tqo_mse_layout* L,
                  uint8_t* pool, int fused_pairsum, int nthreads) {
    kv_ctx c = {key, value, slots, NULL, pool, NULL, NULL, H, D, block_size, fused_pairsum,
                NULL, L};
    parallel_rows((long long)num_tokens * H, nthreads, mse_pack_one, &c);
}

/* B.3 (turbo_mse): cooperative_inverse_transform_and_store, :138-184. */
static void mse_dequant_vec(const uint8_t* codes, float rms, int head, int D, uint16_t* dst) {
    float x[TQO_MAX_D];
    for (int t = 0; t < D / 2; ++t) {
        uint8_t b = codes[t];
        x[2 * t] = kV4[b & 0xf] * rms;
        x[2 * t + 1] = kV4[(b >> 4) & 0xf] * rms;
    }
    tqo_wht(x, D);
    float inv = tqo_inv_sqrt_d(D);
    for (int i = 0; i < D; ++i) dst[i] = tqo_f2h(x[i] * inv * tqo_sign_flip(i, head));
}

static void mse_dequant_one(void* p, long long row) {
    kv_ctx* c = (kv_ctx*)p;
    int t = (int)(row / c->H), h = (int)(row % c->H);
    int slot = c->slots[t];
    if (slot < 0) return;
    int page = slot / c->bs, tib = slot % c->bs, cell = tib * c->H + h;
    const uint8_t* base = c->cpool + (size_t)page * c->ML->page_size;
    const size_t off = (size_t)row * (size_t)c->D;
    float kr = tqo_h2f(get_h(base + c->ML->k_norms_off + (size_t)cell * c->ML->norm_bytes));
    float vr = tqo_h2f(get_h(base + c->ML->v_norms_off + (size_t)cell * c->ML->norm_bytes));
    mse_dequant_vec(base + c->ML->k_codes_off + (size_t)cell * c->ML->code_bytes, kr, h, c->D,
                    c->ok + off);
    mse_dequant_vec(base + c->ML->v_codes_off + (size_t)cell * c->ML->code_bytes, vr, h, c->D,
                    c->ov + off);
}

void tqo_mse_dequant(const uint8_t* pool, const int32_t* slots, int num_tokens, int H, int D,
                     int block_size, const tqo_mse_layout* L, uint16_t* out_key,
                     uint16_t* out_value, int nthreads) {
    kv_ctx c = {NULL, NULL, slots, pool, NULL, out_key, out_value, H, D, block_size, 0, NULL, L};
    parallel_rows((long long)num_tokens * H, nthreads, mse_dequant_one, &c);
}

void tqo_mse_attention_f64(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                           int num_queries, int num_kv_tokens, int H, int D, int block_size,
                           const tqo_mse_layout* L, double* out, int nthreads) {
    att_ctx c = {query, pool, slots, num_queries, num_kv_tokens, H, D, block_size, NULL, L,
                 NULL, out, NULL, NULL};
    parallel_rows((long long)num_queries * H, nthreads, mse_att64_one, &c);
}

void tqo_mse_attention_f32(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                           int num_queries, int num_kv_tokens, int H, int D, int block_size,
                           const tqo_mse_layout* L, uint16_t* out, int nthreads) {
    att_ctx c = {query, pool, slots, num_queries, num_kv_tokens, H, D, block_size, NULL, L,
                 NULL, NULL, NULL, out};
    parallel_rows((long long)num_queries * H, nthreads, mse_att32_one, &c);
}

/* ------------------------------------------------------------------------ */
/* Boundary report                                                           */
/* ------------------------------------------------------------------------ */

static int code_boundary(float x, int (*nearest)(float)) {
    int c0 = nearest(x);
    return nearest(nextafterf(x, INFINITY)) != c0 || nearest(nextafterf(x, -INFINITY)) != c0;
}

void tqo_prod_boundary_count(const uint16_t* key, const uint16_t* value, int num_rows, int H,
                             int D, long long counts[3]) {
    counts[0] = counts[1] = counts[2] = 0;
    float kn[TQO_MAX_D], vn[TQO_MAX_D];
    uint8_t k4[TQO_MAX_D / 2], v4[TQO_MAX_D / 2];
    uint16_t a, b, cc;
    for (int r = 0; r < num_rows; ++r) {
        tqo_prod_pack_row(key + (size_t)r * D, value + (size_t)r * D, r % H, D, k4, v4, &a, &b,
                          &cc, kn, vn);
        for (int i = 0; i < D; ++i) {
            counts[0] += code_boundary(kn[i], tqo_nearest_k3);
            float lvl = kK3[tqo_nearest_k3(kn[i])];
            float up = nextafterf(kn[i], INFINITY) - lvl, dn = nextafterf(kn[i], -INFINITY) - lvl;
            counts[1] += ((up >= 0.0f) != (dn >= 0.0f));
            counts[2] += code_boundary(vn[i], tqo_nearest_v4);
        }
    }
}

/* The values tqo_prod_boundary_count counts, listed: element index
 * row * D + i, kind (0: K code, 1: K residual sign, 2: V code) and the
 * normalised value (kn or vn).  Returns the number found; at most max_out
 * are written. */
long long tqo_prod_boundary_list(const uint16_t* key, const uint16_t* value, int num_rows, int H,
                                 int D, long long* out_elem, int* out_kind, float* out_val,
                                 long long max_out) {
    long long n = 0;
    float kn[TQO_MAX_D], vn[TQO_MAX_D];
    uint8_t k4[TQO_MAX_D / 2], v4[TQO_MAX_D / 2];
    uint16_t a, b, cc;
    for (int r = 0; r < num_rows; ++r) {
        tqo_prod_pack_row(key + (size_t)r * D, value + (size_t)r * D, r % H, D, k4, v4, &a, &b,
                          &cc, kn, vn);
        for (int i = 0; i < D; ++i) {
            float lvl = kK3[tqo_nearest_k3(kn[i])];
            float up = nextafterf(kn[i], INFINITY) - lvl, dn = nextafterf(kn[i], -INFINITY) - lvl;
            const int hit[3] = {code_boundary(kn[i], tqo_nearest_k3), (up >= 0.0f) != (dn >= 0.0f),
                                code_boundary(vn[i], tqo_nearest_v4)};
            for (int kind = 0; kind < 3; ++kind) {
                if (!hit[kind]) continue;
                if (n < max_out) {
                    out_elem[n] = (long long)r * D + i;
                    out_kind[n] = kind;
                    out_val[n] = kind == 2 ? vn[i] : kn[i];
                }
                ++n;
            }
        }
    }
    return n;
}

void tqo_mse_boundary_count(const uint16_t* key, const uint16_t* value, int num_rows, int H,
                            int D, long long counts[3]) {
    counts[0] = counts[1] = counts[2] = 0;
    float xn[TQO_MAX_D];
    uint8_t c1[TQO_MAX_D / 2], c2[TQO_MAX_D / 2];
    uint16_t n1, n2;
    for (int r = 0; r < num_rows; ++r) {
        for (int kv = 0; kv < 2; ++kv) {
            const uint16_t* src = (kv ? value : key) + (size_t)r * D;
            tqo_mse_pack_row(src, r % H, D, 1, c1, &n1, xn);
            tqo_mse_pack_row(src, r % H, D, 0, c2, &n2, NULL);
            for (int i = 0; i < D; ++i) counts[2] += code_boundary(xn[i], tqo_nearest_v4);
            /* counts[0]: rows whose fused and unfused pair-sum disagree on the
             * stored norm; counts[1]: code bytes that differ between the two. */
            counts[0] += (n1 != n2);
            for (int j = 0; j < D / 2; ++j) counts[1] += (c1[j] != c2[j]);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* SDPA oracle — src/tq_attention_ref.cpp:10-56                              */
/* ------------------------------------------------------------------------ */

void tqo_sdpa_single_head(const uint16_t* q, const uint16_t* k_all, const uint16_t* v_all,
                          int num_tokens, int head_dim, float* out) {
    for (int d = 0; d < head_dim; ++d) out[d] = 0.0f;
    if (num_tokens <= 0) return;
    float* sc = (float*)malloc(sizeof(float) * (size_t)num_tokens);
    const float inv = 1.0f / sqrtf((float)head_dim);
    for (int t = 0; t < num_tokens; ++t) {
        float acc = 0.0f;
        for (int d = 0; d < head_dim; ++d)
            acc += tqo_h2f(q[d]) * tqo_h2f(k_all[(size_t)t * head_dim + d]);
        sc[t] = acc * inv;
    }
    float mx = sc[0];
    for (int t = 1; t < num_tokens; ++t)
        if (sc[t] > mx) mx = sc[t];
    float denom = 0.0f;
    for (int t = 0; t < num_tokens; ++t) {
        sc[t] = expf(sc[t] - mx);
        denom += sc[t];
    }
    for (int t = 0; t < num_tokens; ++t) sc[t] /= denom;
    for (int t = 0; t < num_tokens; ++t) {
        float p = sc[t];
        for (int d = 0; d < head_dim; ++d) out[d] += p * tqo_h2f(v_all[(size_t)t * head_dim + d]);
    }
    free(sc);
}

/* ------------------------------------------------------------------------ */
/* Lloyd-Max design — src/gaussian_codebook.cpp:10-83, generalised to M      */
/* ------------------------------------------------------------------------ */

static double npdf(double x) { return 0.39894228040143267794 * exp(-0.5 * x * x); }
static double ncdf(double x) { return 0.5 * erfc(-x / sqrt(2.0)); }

static double trunc_mean(double a, double b) {
    double z = ncdf(b) - ncdf(a);
    if (z <= 1e-15) return 0.5 * (a + b);
    return (npdf(a) - npdf(b)) / z;
}

static double quantile(double p) {
    if (p < 1e-12) p = 1e-12;
    if (p > 1.0 - 1e-12) p = 1.0 - 1e-12;
    double lo = -10.0, hi = 10.0;
    for (int it = 0; it < 120; ++it) {
        double mid = 0.5 * (lo + hi);
        if (ncdf(mid) < p) lo = mid; else hi = mid;
    }
    return 0.5 * (lo + hi);
}

void tqo_lloyd_max_gaussian(int M, int max_iter, double tol, double* levels, double* thr) {
    double c[64] = {0}, t[64] = {0}, cn[64], tn[64];
    if (M < 2 || M > 64) return;
    for (int i = 1; i < M; ++i) t[i - 1] = quantile((double)i / M);
    for (int it = 0; it < max_iter; ++it) {
        for (int i = 0; i < M; ++i) {
            double a = (i == 0) ? -6.0 : t[i - 1];
            double b = (i == M - 1) ? 6.0 : t[i];
            cn[i] = trunc_mean(a, b);
        }
        for (int i = 0; i < M - 1; ++i) tn[i] = 0.5 * (cn[i] + cn[i + 1]);
        double diff = 0.0;
        for (int i = 0; i < M; ++i) diff = fmax(diff, fabs(cn[i] - c[i]));
        for (int i = 0; i < M - 1; ++i) diff = fmax(diff, fabs(tn[i] - t[i]));
        memcpy(c, cn, sizeof(double) * (size_t)M);
        memcpy(t, tn, sizeof(double) * (size_t)(M - 1));
        if (diff < tol) break;
    }
    memcpy(levels, c, sizeof(double) * (size_t)M);
    memcpy(thr, t, sizeof(double) * (size_t)(M - 1));
}

/* ======================================================================== */
/* Kernels the reference compiles but does not export:                      */
/* QJL-1b, the legacy INT4 and dense pages, and the GPU SDPA reference.       */
/* ======================================================================== */

/* src/tq_qjl.cpp:7-33 */
void tqo_make_qjl_layout(int block_size, int H, int D, tqo_qjl_layout* L) {
    memset(L, 0, sizeof(*L));
    L->k1_bytes = (D + 7) / 8;
    L->v4_bytes = (D * 4 + 7) / 8;
    L->scale_bytes = 2;
    size_t th = (size_t)block_size * (size_t)H, cur = 0;
    L->k1_off = cur; cur += th * (size_t)L->k1_bytes;
    cur = align_up(cur, 2);
    L->ks_off = cur; cur += th * 2;
    L->v4_off = cur; cur += th * (size_t)L->v4_bytes;
    cur = align_up(cur, 2);
    L->vs_off = cur; cur += th * 2;
    L->page_size = align_up(cur, 2);
}

/* src/tq_layout.cpp:8-36; returns -1 where the reference throws (nbits != 4,
 * group_size != head_dim).  scale_fp32: TQScaleType::FP32 (4-byte scales). */
int tqo_make_int4_layout(int block_size, int H, int D, int nbits, int group_size,
                         int page_alignment, int scale_fp32, tqo_int4_layout* L) {
    memset(L, 0, sizeof(*L));
    if (nbits != 4 || group_size != D) return -1;
    size_t th = (size_t)block_size * (size_t)H, a = (size_t)page_alignment;
    L->code_bytes = (size_t)D * (size_t)nbits / 8;
    L->scale_bytes = scale_fp32 ? 4 : 2;
    L->k_codes_off = 0;
    L->k_codes_bytes = th * L->code_bytes;
    L->v_codes_off = align_up(L->k_codes_off + L->k_codes_bytes, a);
    L->v_codes_bytes = th * L->code_bytes;
    L->k_scales_off = align_up(L->v_codes_off + L->v_codes_bytes, a);
    L->k_scales_bytes = th * L->scale_bytes;
    L->v_scales_off = align_up(L->k_scales_off + L->k_scales_bytes, a);
    L->v_scales_bytes = th * L->scale_bytes;
    L->page_size = align_up(L->v_scales_off + L->v_scales_bytes, a);
    return 0;
}

/* src/tq_dense_layout.cpp:7-18 */
void tqo_make_dense_layout(int block_size, int H, int D, int page_alignment,
                           tqo_dense_layout* L) {
    memset(L, 0, sizeof(*L));
    size_t th = (size_t)block_size * (size_t)H, a = (size_t)page_alignment;
    L->elem_bytes = 2;
    L->k_off = 0;
    L->k_bytes = th * (size_t)D * 2;
    L->v_off = align_up(L->k_bytes, a);
    L->v_bytes = th * (size_t)D * 2;
    L->page_size = align_up(L->v_off + L->v_bytes, a);
}

/* ---- QJL-1b (src/cuda/tq_qjl_kernels.cu) -------------------------------- */
/* The QJL kernels call sign_flip(idx) without the head (:16-19): (-1)^idx. */
static float qjl_sign(int i) { return tqo_sign_flip(i, 0); }

/* qjl_pack_kv_kernel, :72-181, one (token, head). */
void tqo_qjl_pack_row(const uint16_t* k, const uint16_t* v, int D, uint8_t* k1, uint8_t* v4,
                      uint16_t* ks, uint16_t* vs) {
    float sk[TQO_MAX_D], sv[TQO_MAX_D], red[TQO_MAX_D];
    int bits[TQO_MAX_D], vidx[TQO_MAX_D];
    float inv = tqo_inv_sqrt_d(D);
    for (int i = 0; i < D; ++i) {
        sk[i] = tqo_h2f(k[i]) * qjl_sign(i);
        sv[i] = tqo_h2f(v[i]) * qjl_sign(i);
    }
    tqo_wht(sk, D);
    tqo_wht(sv, D);
    for (int i = 0; i < D; ++i) { sk[i] *= inv; sv[i] *= inv; }
    for (int i = 0; i < D; ++i) red[i] = sk[i] * sk[i];
    float krms = rms_of(red, D, D);
    *ks = tqo_f2h(krms);
    for (int i = 0; i < D; ++i) red[i] = sv[i] * sv[i];
    float vrms = rms_of(red, D, D);
    *vs = tqo_f2h(vrms);
    for (int i = 0; i < D; ++i) {
        bits[i] = (sk[i] / krms >= 0.0f) ? 1 : 0;
        vidx[i] = tqo_nearest_v4(clampf_ref(sv[i] / vrms, -2.75f, 2.75f));
    }
    for (int b = 0; b < (D + 7) / 8; ++b) { /* pack_1bit_byte_from_bits, shared_device :22-31 */
        uint8_t o = 0;
        for (int i = 0; i < 8; ++i)
            if (8 * b + i < D) o |= (uint8_t)((bits[8 * b + i] & 1) << i);
        k1[b] = o;
    }
    for (int j = 0; j < D / 2; ++j) v4[j] = (uint8_t)((vidx[2 * j + 1] << 4) | vidx[2 * j]);
}

typedef struct {
    const uint16_t *k, *v;
    const int32_t* slots;
    int H, D, bs;
    const tqo_qjl_layout* L;
    uint8_t* pool;
    const uint8_t* cpool;
    uint16_t *ok, *ov;
} qjl_ctx;

static void qjl_pack_one(void* p, long long row) {
    qjl_ctx* c = (qjl_ctx*)p;
    int t = (int)(row / c->H), h = (int)(row % c->H);
    int slot = c->slots[t];
    if (slot < 0) return; /* this build's extension: unmapped token */
    int page = slot / c->bs, tib = slot % c->bs;
    size_t cell = (size_t)tib * c->H + h;
    uint8_t* base = c->pool + (size_t)page * c->L->page_size;
    uint16_t ks, vs;
    const size_t off = (size_t)row * c->D;
    tqo_qjl_pack_row(c->k + off, c->v + off, c->D, base + c->L->k1_off + cell * c->L->k1_bytes,
                     base + c->L->v4_off + cell * c->L->v4_bytes, &ks, &vs);
    put_h(base + c->L->ks_off + cell * 2, ks);
    put_h(base + c->L->vs_off + cell * 2, vs);
}

void tqo_qjl_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                  int num_tokens, int H, int D, int block_size, const tqo_qjl_layout* L,
                  uint8_t* pool, int nthreads) {
    qjl_ctx c = {key, value, slots, H, D, block_size, L, pool, NULL, NULL, NULL};
    parallel_rows((long long)num_tokens * H, nthreads, qjl_pack_one, &c);
}

static int bit_get(const uint8_t* src, int i) { return (src[i >> 3] >> (i & 7)) & 1; }

typedef struct {
    const uint8_t *k1, *v4;
    float ks, vs;
} qjl_cell_t;

static void qjl_cell(const uint8_t* pool, const int32_t* slots, int t, int h, int H, int bs,
                     const tqo_qjl_layout* L, qjl_cell_t* o) {
    int slot = slots[t], page = slot / bs, tib = slot % bs;
    size_t cell = (size_t)tib * H + h;
    const uint8_t* base = pool + (size_t)page * L->page_size;
    o->k1 = base + L->k1_off + cell * L->k1_bytes;
    o->v4 = base + L->v4_off + cell * L->v4_bytes;
    o->ks = tqo_h2f(get_h(base + L->ks_off + cell * 2));
    o->vs = tqo_h2f(get_h(base + L->vs_off + cell * 2));
}

/* qjl_dequant_kv_kernel, :189-245. */
static void qjl_dequant_one(void* p, long long row) {
    qjl_ctx* c = (qjl_ctx*)p;
    int t = (int)(row / c->H), h = (int)(row % c->H), D = c->D;
    if (c->slots[t] < 0) return;
    qjl_cell_t ce;
    qjl_cell(c->cpool, c->slots, t, h, c->H, c->bs, c->L, &ce);
    float sk[TQO_MAX_D], sv[TQO_MAX_D];
    for (int i = 0; i < D; ++i) {
        sk[i] = (bit_get(ce.k1, i) ? 1.0f : -1.0f) * ce.ks;
        sv[i] = kV4[nib_get(ce.v4, i)] * ce.vs;
    }
    tqo_wht(sk, D);
    tqo_wht(sv, D);
    float inv = tqo_inv_sqrt_d(D);
    for (int i = 0; i < D; ++i) {
        c->ok[(size_t)row * D + i] = tqo_f2h(sk[i] * inv * qjl_sign(i));
        c->ov[(size_t)row * D + i] = tqo_f2h(sv[i] * inv * qjl_sign(i));
    }
}

void tqo_qjl_dequant(const uint8_t* pool, const int32_t* slots, int num_tokens, int H, int D,
                     int block_size, const tqo_qjl_layout* L, uint16_t* out_key,
                     uint16_t* out_value, int nthreads) {
    qjl_ctx c = {NULL, NULL, slots, H, D, block_size, L, NULL, pool, out_key, out_value};
    parallel_rows((long long)num_tokens * H, nthreads, qjl_dequant_one, &c);
}

typedef struct {
    const uint16_t* q;
    const uint8_t* pool;
    const int32_t* slots;
    int Q, N, H, D, bs;
    const tqo_qjl_layout* L;
    double* out_d;
    uint16_t* out_h;
} qjl_att_ctx;

/* Exact: logit = <qrot, +-ks> (no 1/sqrt(D), :254 "Logit convention"),
 * softmax, acc = sum p * vs * V4, acc / l, inverse WHT, * s_i / sqrt(D). */
static void qjl_att64_one(void* p, long long row) {
    qjl_att_ctx* c = (qjl_att_ctx*)p;
    int qi = (int)(row / c->H), h = (int)(row % c->H), D = c->D, N = c->N;
    float qrot[TQO_MAX_D];
    double qd[TQO_MAX_D], acc[TQO_MAX_D];
    float inv = tqo_inv_sqrt_d(D);
    const uint16_t* q = c->q + ((size_t)qi * c->H + h) * (size_t)D;
    for (int i = 0; i < D; ++i) qrot[i] = tqo_h2f(q[i]) * qjl_sign(i);
    tqo_wht(qrot, D);
    for (int i = 0; i < D; ++i) { qd[i] = (double)(qrot[i] * inv); acc[i] = 0.0; }
    double* lg = (double*)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
    double mx = -INFINITY;
    for (int t = 0; t < N; ++t) {
        if (c->slots[t] < 0) { lg[t] = -INFINITY; continue; }
        qjl_cell_t ce;
        qjl_cell(c->pool, c->slots, t, h, c->H, c->bs, c->L, &ce);
        double s = 0.0;
        for (int i = 0; i < D; ++i) s += bit_get(ce.k1, i) ? qd[i] : -qd[i];
        lg[t] = s * (double)ce.ks;
        if (lg[t] > mx) mx = lg[t];
    }
    double l = 0.0;
    for (int t = 0; t < N; ++t) {
        if (c->slots[t] < 0) continue;
        qjl_cell_t ce;
        qjl_cell(c->pool, c->slots, t, h, c->H, c->bs, c->L, &ce);
        double w = exp(lg[t] - mx);
        l += w;
        for (int i = 0; i < D; ++i) acc[i] += w * (double)ce.vs * (double)kV4[nib_get(ce.v4, i)];
    }
    free(lg);
    if (l > 0.0)
        for (int i = 0; i < D; ++i) acc[i] /= l;
    wht_f64(acc, D);
    double invd = 1.0 / sqrt((double)D);
    double* o = c->out_d + ((size_t)qi * c->H + h) * (size_t)D;
    for (int i = 0; i < D; ++i) o[i] = acc[i] * invd * (double)qjl_sign(i);
}

/* qjl_fused_attn_online_kernel, :262-378, in fp32 in the kernel's order. */
static void qjl_att32_one(void* p, long long row) {
    qjl_att_ctx* c = (qjl_att_ctx*)p;
    int qi = (int)(row / c->H), h = (int)(row % c->H), D = c->D;
    float qrot[TQO_MAX_D], vacc[TQO_MAX_D], red[TQO_MAX_D];
    float inv = tqo_inv_sqrt_d(D);
    const uint16_t* q = c->q + ((size_t)qi * c->H + h) * (size_t)D;
    for (int i = 0; i < D; ++i) qrot[i] = tqo_h2f(q[i]) * qjl_sign(i);
    tqo_wht(qrot, D);
    for (int i = 0; i < D; ++i) { qrot[i] *= inv; vacc[i] = 0.0f; }
    float m = -1e30f, l = 0.0f;
    for (int t = 0; t < c->N; ++t) {
        if (c->slots[t] < 0) continue;
        qjl_cell_t ce;
        qjl_cell(c->pool, c->slots, t, h, c->H, c->bs, c->L, &ce);
        for (int i = 0; i < D; ++i) red[i] = qrot[i] * ((bit_get(ce.k1, i) ? 1.0f : -1.0f) * ce.ks);
        float logit = tqo_tree_sum(red, D);
        float m_new = fmaxf(m, logit);
        float a = expf(m - m_new), b = expf(logit - m_new);
        l = l * a + b;
        m = m_new;
        for (int i = 0; i < D; ++i) {
            vacc[i] *= a;
            vacc[i] += b * (kV4[nib_get(ce.v4, i)] * ce.vs);
        }
    }
    float inv_l = (l > 0.0f) ? (1.0f / l) : 1.0f;
    for (int i = 0; i < D; ++i) vacc[i] *= inv_l;
    tqo_wht(vacc, D);
    uint16_t* o = c->out_h + ((size_t)qi * c->H + h) * (size_t)D;
    for (int i = 0; i < D; ++i) o[i] = tqo_f2h(vacc[i] * inv * qjl_sign(i));
}

void tqo_qjl_attention_f64(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                           int num_queries, int num_kv_tokens, int H, int D, int block_size,
                           const tqo_qjl_layout* L, double* out, int nthreads) {
    qjl_att_ctx c = {query, pool, slots, num_queries, num_kv_tokens, H, D, block_size, L, out, NULL};
    parallel_rows((long long)num_queries * H, nthreads, qjl_att64_one, &c);
}

void tqo_qjl_attention_f32(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                           int num_queries, int num_kv_tokens, int H, int D, int block_size,
                           const tqo_qjl_layout* L, uint16_t* out, int nthreads) {
    qjl_att_ctx c = {query, pool, slots, num_queries, num_kv_tokens, H, D, block_size, L, NULL, out};
    parallel_rows((long long)num_queries * H, nthreads, qjl_att32_one, &c);
}

/* ---- legacy INT4 (src/cuda/tq_pack_kernels.cu, tq_dequant_kernels.cu) ---- */

/* __float2int_rn: round half to even; NaN converts to 0 (PTX cvt.rni). */
static int f2i_rn(float x) {
    if (x != x) return 0;
    float r = rintf(x);
    if (r >= 2147483647.0f) return 2147483647;
    if (r <= -2147483648.0f) return (-2147483647 - 1);
    return (int)r;
}

/* quantize_to_int4, tq_pack_kernels.cu:30-34 */
static int q_int4(float x, float scale) {
    if (scale <= 1e-12f) return 0;
    int q = f2i_rn(x / scale);
    return q < -8 ? -8 : (q > 7 ? 7 : q);
}

/* tq_pack_kv_kernel, :36-110, one (token, head): scale = max(absmax / 7, 1e-8)
 * (fp32; the fp16 copy is what is stored), codes two's-complement nibbles. */
void tqo_int4_pack_row(const uint16_t* k, const uint16_t* v, int D, uint8_t* kc, uint8_t* vc,
                       uint16_t* ks, uint16_t* vs) {
    float ka = 0.0f, va = 0.0f;
    for (int i = 0; i < D; ++i) {
        ka = fmaxf(ka, fabsf(tqo_h2f(k[i])));
        va = fmaxf(va, fabsf(tqo_h2f(v[i])));
    }
    float kscale = fmaxf(ka / 7.0f, 1e-8f), vscale = fmaxf(va / 7.0f, 1e-8f);
    *ks = tqo_f2h(kscale);
    *vs = tqo_f2h(vscale);
    for (int i = 0; i < D; i += 2) {
        int k0 = q_int4(tqo_h2f(k[i]), kscale), v0 = q_int4(tqo_h2f(v[i]), vscale);
        int k1 = 0, v1 = 0;
        if (i + 1 < D) {
            k1 = q_int4(tqo_h2f(k[i + 1]), kscale);
            v1 = q_int4(tqo_h2f(v[i + 1]), vscale);
        }
        kc[i / 2] = (uint8_t)((k0 & 0xF) | ((k1 & 0xF) << 4)); /* pack_int4, tq_quant.h:8-10 */
        vc[i / 2] = (uint8_t)((v0 & 0xF) | ((v1 & 0xF) << 4));
    }
}

typedef struct {
    const uint16_t *k, *v;
    const int32_t* slots;
    int H, D, bs;
    const tqo_int4_layout* L;
    uint8_t* pool;
    const uint8_t* cpool;
    uint16_t *ok, *ov;
} int4_ctx;

static void int4_pack_one(void* p, long long row) {
    int4_ctx* c = (int4_ctx*)p;
    int t = (int)(row / c->H), h = (int)(row % c->H), slot = c->slots[t];
    if (slot < 0) return;
    int page = slot / c->bs, tib = slot % c->bs;
    size_t cell = (size_t)tib * c->H + h;
    uint8_t* base = c->pool + (size_t)page * c->L->page_size;
    uint16_t ks, vs;
    tqo_int4_pack_row(c->k + (size_t)row * c->D, c->v + (size_t)row * c->D, c->D,
                      base + c->L->k_codes_off + cell * c->L->code_bytes,
                      base + c->L->v_codes_off + cell * c->L->code_bytes, &ks, &vs);
    /* a half at the scale cell, whatever the cell size (:84-88) */
    put_h(base + c->L->k_scales_off + cell * c->L->scale_bytes, ks);
    put_h(base + c->L->v_scales_off + cell * c->L->scale_bytes, vs);
}

void tqo_int4_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                   int num_tokens, int H, int D, int block_size, const tqo_int4_layout* L,
                   uint8_t* pool, int nthreads) {
    int4_ctx c = {key, value, slots, H, D, block_size, L, pool, NULL, NULL, NULL};
    parallel_rows((long long)num_tokens * H, nthreads, int4_pack_one, &c);
}

static int s4(int n) { return n >= 8 ? n - 16 : n; } /* unpack_int4_low/high, tq_quant.h:12-20 */

/* tq_dequant_kv_kernel, tq_dequant_kernels.cu:6-55: f2h(q * f32(scale)). */
static void int4_dequant_one(void* p, long long row) {
    int4_ctx* c = (int4_ctx*)p;
    int t = (int)(row / c->H), h = (int)(row % c->H), slot = c->slots[t], D = c->D;
    if (slot < 0) return;
    int page = slot / c->bs, tib = slot % c->bs;
    size_t cell = (size_t)tib * c->H + h;
    const uint8_t* base = c->cpool + (size_t)page * c->L->page_size;
    const uint8_t* kc = base + c->L->k_codes_off + cell * c->L->code_bytes;
    const uint8_t* vc = base + c->L->v_codes_off + cell * c->L->code_bytes;
    float ks = tqo_h2f(get_h(base + c->L->k_scales_off + cell * c->L->scale_bytes));
    float vs = tqo_h2f(get_h(base + c->L->v_scales_off + cell * c->L->scale_bytes));
    for (int i = 0; i < D; ++i) {
        int kn = (i & 1) ? kc[i / 2] >> 4 : kc[i / 2] & 0xF;
        int vn = (i & 1) ? vc[i / 2] >> 4 : vc[i / 2] & 0xF;
        c->ok[(size_t)row * D + i] = tqo_f2h((float)s4(kn) * ks);
        c->ov[(size_t)row * D + i] = tqo_f2h((float)s4(vn) * vs);
    }
}

void tqo_int4_dequant(const uint8_t* pool, const int32_t* slots, int num_tokens, int H, int D,
                      int block_size, const tqo_int4_layout* L, uint16_t* out_key,
                      uint16_t* out_value, int nthreads) {
    int4_ctx c = {NULL, NULL, slots, H, D, block_size, L, NULL, pool, out_key, out_value};
    parallel_rows((long long)num_tokens * H, nthreads, int4_dequant_one, &c);
}

/* ---- GPU SDPA reference (src/cuda/tq_attention_ref_kernel.cu:24-112) ----- */
/* Per (query, head): logits = tree-sum(q * k) * inv into logit_scratch, max,
 * sum of expf in token order, 1/sum, then V accumulated in token order with
 * weight expf(l - max) * (1/sum); fp16 output.  fp32 throughout. */
typedef struct {
    const uint16_t *q, *k, *v;
    uint16_t* out;
    float* logits;
    int Q, N, H, D;
} sdpa_ctx;

static void sdpa_gpu_one(void* p, long long row) {
    sdpa_ctx* c = (sdpa_ctx*)p;
    int qi = (int)(row / c->H), h = (int)(row % c->H), D = c->D, N = c->N;
    float q[TQO_MAX_D], red[TQO_MAX_D], vacc[TQO_MAX_D];
    float inv = tqo_inv_sqrt_d(D);
    for (int i = 0; i < D; ++i) q[i] = tqo_h2f(c->q[((size_t)qi * c->H + h) * D + i]);
    float* lg = c->logits + ((size_t)qi * c->H + h) * (size_t)N;
    float mx = -1e30f;
    for (int t = 0; t < N; ++t) {
        const uint16_t* kr = c->k + ((size_t)t * c->H + h) * D;
        for (int i = 0; i < D; ++i) red[i] = q[i] * tqo_h2f(kr[i]);
        float logit = tqo_tree_sum(red, D) * inv;
        lg[t] = logit;
        if (logit > mx) mx = logit;
    }
    float s = 0.0f;
    for (int t = 0; t < N; ++t) s += expf(lg[t] - mx);
    float inv_sum = (s > 0.0f) ? (1.0f / s) : 1.0f;
    for (int i = 0; i < D; ++i) vacc[i] = 0.0f;
    for (int t = 0; t < N; ++t) {
        float w = expf(lg[t] - mx) * inv_sum;
        const uint16_t* vr = c->v + ((size_t)t * c->H + h) * D;
        for (int i = 0; i < D; ++i) vacc[i] += w * tqo_h2f(vr[i]);
    }
    for (int i = 0; i < D; ++i) c->out[((size_t)qi * c->H + h) * D + i] = tqo_f2h(vacc[i]);
}

void tqo_sdpa_gpu_ref(const uint16_t* query, const uint16_t* key, const uint16_t* value,
                      uint16_t* out, float* logits, int num_queries, int num_kv_tokens, int H,
                      int D, int nthreads) {
    sdpa_ctx c = {query, key, value, out, logits, num_queries, num_kv_tokens, H, D};
    parallel_rows((long long)num_queries * H, nthreads, sdpa_gpu_one, &c);
}

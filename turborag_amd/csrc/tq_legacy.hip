// tq_legacy.hip — the kernels the reference compiles but does not export,
// for gfx950: QJL-1b pack / dequant / fused attention
// (src/cuda/tq_qjl_kernels.cu), the legacy INT4 page pack / dequant
// (src/cuda/tq_pack_kernels.cu, tq_dequant_kernels.cu), the dense fp16 page
// store / load (src/cuda/tq_dense_kernels.cu) and the GPU SDPA reference
// (src/cuda/tq_attention_ref_kernel.cu).
//
// Rows follow the row convention of tq_device.h (one (token, head) vector on
// D/2 lanes, two elements per lane), so the QJL rotation and RMS trees are
// the reference's float operations in its order (bit-exact codes, scales and
// dequantized halves).  QJL attention is split-K with a combine, like the
// turbo kernels' generic path; the SDPA reference splits its token passes
// over the waves of a workgroup.  Tokens with a negative slot are skipped.
#include <algorithm>

#include "tq_device.h"

namespace tq {
namespace {

using namespace dev;

constexpr int kBlock = 256;
constexpr float kInitMax = -1e30f;  // include/tq_shared_device.cuh:10

__device__ __forceinline__ void page_of(int slot, int block_size, int& page, int& tib) {
    page = slot / block_size;
    tib = slot - page * block_size;
}

__device__ __forceinline__ void put_u16(uint8_t* p, uint16_t v) {
    *reinterpret_cast<uint16_t*>(p) = v;
}

// ---------------------------------------------------------------------------
// QJL-1b.  The QJL kernels call sign_flip(idx) without the head (:16-19):
// element i has sign (-1)^i, so in lane j element 2j keeps its sign and
// 2j + 1 is negated.
// ---------------------------------------------------------------------------

// qjl_pack_kv_kernel (:72-181): rotate, RMS of K and V, K sign bits
// (x / rms >= 0), V nearest 4-bit level of clamp(x / rms, +-2.75).
template <int D>
__global__ __launch_bounds__(kBlock) void qjl_pack_kernel(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
    const int32_t* __restrict__ slots, uint8_t* __restrict__ pool, QjlGeom g, int num_rows,
    float inv) {
    constexpr int L = D / 2;
    const int j = threadIdx.x % L;
    const int row = blockIdx.x * (kBlock / L) + threadIdx.x / L;
    const bool valid = row < num_rows;
    const int rr = valid ? row : num_rows - 1;
    const int t = rr / g.H, h = rr - t * g.H;
    const size_t off = (size_t)rr * D + 2 * j;
    const uint32_t kk = *reinterpret_cast<const uint32_t*>(key + off);
    const uint32_t vv = *reinterpret_cast<const uint32_t*>(value + off);
    float k0 = h2f(kk & 0xffff), k1 = -h2f(kk >> 16);
    float v0 = h2f(vv & 0xffff), v1 = -h2f(vv >> 16);
    wht_pair<L>(k0, k1, j);
    wht_pair<L>(v0, v1, j);
    k0 *= inv; k1 *= inv; v0 *= inv; v1 *= inv;
    float krms = sqrtf(tree_pair<L>(k0 * k0, k1 * k1) / (float)D);
    if (krms < kMinRMS) krms = kMinRMS;
    float vrms = sqrtf(tree_pair<L>(v0 * v0, v1 * v1) / (float)D);
    if (vrms < kMinRMS) vrms = kMinRMS;
    const uint32_t b0 = (k0 / krms >= 0.0f) ? 1u : 0u, b1 = (k1 / krms >= 0.0f) ? 1u : 0u;
    const int q0 = nearest_v4(clamp_ref(v0 / vrms, -2.75f, 2.75f));
    const int q1 = nearest_v4(clamp_ref(v1 / vrms, -2.75f, 2.75f));
    // Bits 2j, 2j+1 of the row are bits 2(j%4), 2(j%4)+1 of byte j/4: OR the
    // quad of lanes (all of one row when L >= 4; D = 2, 4 have one byte).
    uint32_t bits = (b0 | (b1 << 1)) << (2 * (j & 3));
    if constexpr (L >= 2) bits |= __float_as_uint(quad_xor<1>(__uint_as_float(bits)));
    if constexpr (L >= 4) bits |= __float_as_uint(quad_xor<2>(__uint_as_float(bits)));
    if (!valid) return;
    const int slot = slots[t];
    if (slot < 0) return;
    int page, tib;
    page_of(slot, g.block_size, page, tib);
    const size_t cell = (size_t)tib * g.H + h;
    uint8_t* base = pool + (size_t)page * g.page_size;
    if ((j & 3) == 0) base[g.k1_off + cell * g.k1_bytes + (j >> 2)] = (uint8_t)bits;
    base[g.v4_off + cell * g.v4_bytes + j] = (uint8_t)(q0 | (q1 << 4));
    if (j == 0) {
        put_u16(base + g.ks_off + cell * 2, f2h(krms));
        put_u16(base + g.vs_off + cell * 2, f2h(vrms));
    }
}

// qjl_dequant_kv_kernel (:189-245): (+-1) * ks and V4[c] * vs in the rotated
// domain, WHT, then * (1/sqrt(D)) * sign.
template <int D>
__global__ __launch_bounds__(kBlock) void qjl_dequant_kernel(
    const uint8_t* __restrict__ pool, const int32_t* __restrict__ slots,
    uint16_t* __restrict__ out_key, uint16_t* __restrict__ out_value, QjlGeom g, int num_rows,
    float inv) {
    constexpr int L = D / 2;
    const int j = threadIdx.x % L;
    const int row = blockIdx.x * (kBlock / L) + threadIdx.x / L;
    const bool valid = row < num_rows;
    const int rr = valid ? row : num_rows - 1;
    const int t = rr / g.H, h = rr - t * g.H;
    const int slot = slots[t];
    float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
    if (slot >= 0) {
        int page, tib;
        page_of(slot, g.block_size, page, tib);
        const size_t cell = (size_t)tib * g.H + h;
        const uint8_t* base = pool + (size_t)page * g.page_size;
        const uint32_t kb = base[g.k1_off + cell * g.k1_bytes + (j >> 2)] >> (2 * (j & 3));
        const uint32_t vb = base[g.v4_off + cell * g.v4_bytes + j];
        const float ks = h2f(ld_u16(base + g.ks_off + cell * 2));
        const float vs = h2f(ld_u16(base + g.vs_off + cell * 2));
        k0 = ((kb & 1) ? 1.0f : -1.0f) * ks;
        k1 = ((kb & 2) ? 1.0f : -1.0f) * ks;
        v0 = pick(kV4, vb & 0xf) * vs;
        v1 = pick(kV4, vb >> 4) * vs;
    }
    wht_pair<L>(k0, k1, j);
    wht_pair<L>(v0, v1, j);
    if (!valid || slot < 0) return;
    const size_t off = (size_t)rr * D + 2 * j;
    *reinterpret_cast<uint32_t*>(out_key + off) = f2h2(k0 * inv, -(k1 * inv));
    *reinterpret_cast<uint32_t*>(out_value + off) = f2h2(v0 * inv, -(v1 * inv));
}

// QJL attention, split-K partial: one wave per (split, row = q*H + h).  The
// rotated query qrot = WHT(q * s) * inv; logit = <qrot, (+-1) * ks> (no
// 1/sqrt(D), :254); online softmax with expf; V accumulated in the rotated
// domain.  ws[(split * rows + row) * (D + 2) + ...] = acc[0..D), m, l.
template <int D>
__global__ __launch_bounds__(64) void qjl_attn_partial_kernel(
    const uint16_t* __restrict__ query, const uint8_t* __restrict__ pool,
    const int32_t* __restrict__ slots, float* __restrict__ ws, QjlGeom g, int rows,
    int num_kv_tokens, int tokens_per_split, int num_splits, float inv) {
    constexpr int L = D / 2;
    const int lane = threadIdx.x, j = lane % L;
    const int split = blockIdx.x % num_splits;
    const int row = blockIdx.x / num_splits;
    const int h = row % g.H;
    const uint32_t qq = *reinterpret_cast<const uint32_t*>(query + (size_t)row * D + 2 * j);
    float q0 = h2f(qq & 0xffff), q1 = -h2f(qq >> 16);
    wht_pair<L>(q0, q1, j);
    q0 *= inv;
    q1 *= inv;
    const int t0 = split * tokens_per_split;
    const int t1 = min(num_kv_tokens, t0 + tokens_per_split);
    float m = kInitMax, l = 0.0f, a0 = 0.0f, a1 = 0.0f;
    for (int t = t0; t < t1; ++t) {
        const int slot = slots[t];
        if (slot < 0) continue;  // unmapped token (wave-uniform)
        int page, tib;
        page_of(slot, g.block_size, page, tib);
        const size_t cell = (size_t)tib * g.H + h;
        const uint8_t* base = pool + (size_t)page * g.page_size;
        const uint32_t kb = base[g.k1_off + cell * g.k1_bytes + (j >> 2)] >> (2 * (j & 3));
        const float ks = h2f(ld_u16(base + g.ks_off + cell * 2));
        const float s = ((kb & 1) ? q0 : -q0) + ((kb & 2) ? q1 : -q1);
        const float logit = sum_lanes<L>(s) * ks;
        const float m_new = fmaxf(m, logit);
        const float a = expf(m - m_new), b = expf(logit - m_new);
        l = l * a + b;
        m = m_new;
        const uint32_t vb = base[g.v4_off + cell * g.v4_bytes + j];
        const float vs = h2f(ld_u16(base + g.vs_off + cell * 2));
        a0 = a0 * a + b * (pick(kV4, vb & 0xf) * vs);
        a1 = a1 * a + b * (pick(kV4, vb >> 4) * vs);
    }
    float* out = ws + ((size_t)split * rows + row) * (D + 2);
    if (lane < L) {
        out[2 * j] = a0;
        out[2 * j + 1] = a1;
    }
    if (lane == 0) {
        out[D] = m;
        out[D + 1] = l;
    }
}

// Merge the splits, * (1/l), inverse WHT, * inv * sign, fp16 (:364-377).
template <int D>
__global__ __launch_bounds__(64) void qjl_attn_combine_kernel(const float* __restrict__ ws,
                                                              uint16_t* __restrict__ output,
                                                              int rows, int num_splits,
                                                              float inv) {
    constexpr int L = D / 2;
    const int lane = threadIdx.x, j = lane % L;
    const int row = blockIdx.x;
    float M = kInitMax;
    for (int s = 0; s < num_splits; ++s) M = fmaxf(M, ws[((size_t)s * rows + row) * (D + 2) + D]);
    float lsum = 0.0f, a0 = 0.0f, a1 = 0.0f;
    for (int s = 0; s < num_splits; ++s) {
        const float* p = ws + ((size_t)s * rows + row) * (D + 2);
        const float w = expf(p[D] - M);
        lsum += p[D + 1] * w;
        a0 += p[2 * j] * w;
        a1 += p[2 * j + 1] * w;
    }
    const float inv_l = lsum > 0.0f ? 1.0f / lsum : 1.0f;
    a0 *= inv_l;
    a1 *= inv_l;
    wht_pair<L>(a0, a1, j);
    if (lane >= L) return;
    *reinterpret_cast<uint32_t*>(output + (size_t)row * D + 2 * j) =
        f2h2(a0 * inv, -(a1 * inv));
}

// ---------------------------------------------------------------------------
// Legacy INT4 page (no rotation): scale = max(absmax / 7, 1e-8) per
// (token, head), codes = clamp(rint(x / scale), -8, 7) as two's-complement
// nibbles, the fp16 scale stored at the start of the scale cell.
// ---------------------------------------------------------------------------

// quantize_to_int4, tq_pack_kernels.cu:30-34 (__float2int_rn: half to even;
// NaN converts to 0).
__device__ __forceinline__ int q_int4(float x, float scale) {
    if (scale <= 1e-12f) return 0;
    const float r = __builtin_rintf(x / scale);
    if (r != r) return 0;
    return (int)fminf(fmaxf(r, -8.0f), 7.0f);
}

// tq_pack_kv_kernel, tq_pack_kernels.cu:36-110.
template <int D>
__global__ __launch_bounds__(kBlock) void int4_pack_kernel(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
    const int32_t* __restrict__ slots, uint8_t* __restrict__ pool, Int4Geom g, int num_rows) {
    constexpr int L = D / 2;
    const int j = threadIdx.x % L;
    const int row = blockIdx.x * (kBlock / L) + threadIdx.x / L;
    const bool valid = row < num_rows;
    const int rr = valid ? row : num_rows - 1;
    const int t = rr / g.H, h = rr - t * g.H;
    const size_t off = (size_t)rr * D + 2 * j;
    const uint32_t kk = *reinterpret_cast<const uint32_t*>(key + off);
    const uint32_t vv = *reinterpret_cast<const uint32_t*>(value + off);
    const float k0 = h2f(kk & 0xffff), k1 = h2f(kk >> 16);
    const float v0 = h2f(vv & 0xffff), v1 = h2f(vv >> 16);
    // absmax over the row (fmaxf from 0 ignores NaN, as block_max does)
    float ka = fmaxf(fmaxf(0.0f, fabsf(k0)), fabsf(k1));
    float va = fmaxf(fmaxf(0.0f, fabsf(v0)), fabsf(v1));
#pragma unroll
    for (int m = L / 2; m >= 1; m >>= 1) {
        ka = fmaxf(ka, xor_lane(ka, m));
        va = fmaxf(va, xor_lane(va, m));
    }
    const float kscale = fmaxf(ka / 7.0f, 1e-8f), vscale = fmaxf(va / 7.0f, 1e-8f);
    if (!valid) return;
    const int slot = slots[t];
    if (slot < 0) return;
    int page, tib;
    page_of(slot, g.block_size, page, tib);
    const size_t cell = (size_t)tib * g.H + h;
    uint8_t* base = pool + (size_t)page * g.page_size;
    base[g.kc_off + cell * g.code_bytes + j] =
        (uint8_t)((q_int4(k0, kscale) & 0xF) | ((q_int4(k1, kscale) & 0xF) << 4));
    base[g.vc_off + cell * g.code_bytes + j] =
        (uint8_t)((q_int4(v0, vscale) & 0xF) | ((q_int4(v1, vscale) & 0xF) << 4));
    if (j == 0) {
        put_u16(base + g.ks_off + cell * g.scale_bytes, f2h(kscale));
        put_u16(base + g.vs_off + cell * g.scale_bytes, f2h(vscale));
    }
}

// The same for D = 128, wide: 16 lanes per (token, head) row, lane j owns
// elements 8j .. 8j + 7 (one 16-byte load, one code dword).  The row's scale
// is one correctly rounded division; x / scale is Markstein's FMA-corrected
// product with its reciprocal (div_by: correctly rounded for these ranges,
// quotients of |x| <= 65504 by scale >= 1e-8, or zero), then rounded half to
// even, NaN to 0, clamped to [-8, 7].
__device__ __forceinline__ uint32_t q_int4_pair(float x0, float x1, float scale, float y) {
    auto q = [&](float x) {
        float r = __builtin_rintf(div_by(x, scale, y));
        r = r == r ? r : 0.0f;  // NaN (a non-finite x or scale) converts to 0
        return (uint32_t)(int)fminf(fmaxf(r, -8.0f), 7.0f) & 0xFu;
    };
    return q(x0) | (q(x1) << 4);
}

typedef uint16_t h8v __attribute__((ext_vector_type(8)));
__global__ __launch_bounds__(kBlock) void int4_pack_wide_kernel(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
    const int32_t* __restrict__ slots, uint8_t* __restrict__ pool, Int4Geom g, int num_rows) {
    constexpr int D = 128;
    const int j = threadIdx.x & 15;
    const int row = blockIdx.x * (kBlock / 16) + (threadIdx.x >> 4);
    const bool valid = row < num_rows;
    const int rr = valid ? row : num_rows - 1;
    const int t = rr / g.H, h = rr - t * g.H;
    const size_t off = (size_t)rr * D + 8 * j;
    const h8v kr = *reinterpret_cast<const h8v*>(key + off);
    const h8v vr = *reinterpret_cast<const h8v*>(value + off);
    float k[8], v[8];
    // absmax over the row (fmaxf from 0 ignores NaN, as block_max does)
    float ka = 0.0f, va = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        k[e] = h2f(kr[e]);
        v[e] = h2f(vr[e]);
        ka = fmaxf(ka, fabsf(k[e]));
        va = fmaxf(va, fabsf(v[e]));
    }
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) {
        ka = fmaxf(ka, xor_lane(ka, m));
        va = fmaxf(va, xor_lane(va, m));
    }
    const float kscale = fmaxf(ka / 7.0f, 1e-8f), vscale = fmaxf(va / 7.0f, 1e-8f);
    const float ky = 1.0f / kscale, vy = 1.0f / vscale;
    uint32_t kw = 0, vw = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        kw |= q_int4_pair(k[2 * b], k[2 * b + 1], kscale, ky) << (8 * b);
        vw |= q_int4_pair(v[2 * b], v[2 * b + 1], vscale, vy) << (8 * b);
    }
    if (!valid) return;
    const int slot = slots[t];
    if (slot < 0) return;
    int page, tib;
    page_of(slot, g.block_size, page, tib);
    const size_t cell = (size_t)tib * g.H + h;
    uint8_t* base = pool + (size_t)page * g.page_size;
    reinterpret_cast<uint32_t*>(base + g.kc_off + cell * g.code_bytes)[j] = kw;
    reinterpret_cast<uint32_t*>(base + g.vc_off + cell * g.code_bytes)[j] = vw;
    if (j == 0) {
        put_u16(base + g.ks_off + cell * g.scale_bytes, f2h(kscale));
        put_u16(base + g.vs_off + cell * g.scale_bytes, f2h(vscale));
    }
}

// tq_dequant_kv_kernel, tq_dequant_kernels.cu:6-55: fp16(code * fp32(scale)).
template <int D>
__global__ __launch_bounds__(kBlock) void int4_dequant_kernel(
    const uint8_t* __restrict__ pool, const int32_t* __restrict__ slots,
    uint16_t* __restrict__ out_key, uint16_t* __restrict__ out_value, Int4Geom g,
    int num_rows) {
    constexpr int L = D / 2;
    const int j = threadIdx.x % L;
    const int row = blockIdx.x * (kBlock / L) + threadIdx.x / L;
    if (row >= num_rows) return;
    const int t = row / g.H, h = row - t * g.H;
    const int slot = slots[t];
    if (slot < 0) return;
    int page, tib;
    page_of(slot, g.block_size, page, tib);
    const size_t cell = (size_t)tib * g.H + h;
    const uint8_t* base = pool + (size_t)page * g.page_size;
    const int kb = base[g.kc_off + cell * g.code_bytes + j];
    const int vb = base[g.vc_off + cell * g.code_bytes + j];
    const float ks = h2f(ld_u16(base + g.ks_off + cell * g.scale_bytes));
    const float vs = h2f(ld_u16(base + g.vs_off + cell * g.scale_bytes));
    const auto s4 = [](int n) { return (float)(n >= 8 ? n - 16 : n); };
    const size_t off = (size_t)row * D + 2 * j;
    *reinterpret_cast<uint32_t*>(out_key + off) = f2h2(s4(kb & 0xF) * ks, s4(kb >> 4) * ks);
    *reinterpret_cast<uint32_t*>(out_value + off) = f2h2(s4(vb & 0xF) * vs, s4(vb >> 4) * vs);
}

// The same for D = 128, streaming: 16 lanes per (token, head) row, four rows
// per wave.  Lane j decodes code dword j (elements 8j .. 8j + 7: a nibble
// sign-extends with one bit-field extract) and writes 16 bytes, so each
// tensor's row of 256 bytes leaves as two whole 128-byte lines in one
// non-temporal store instruction.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(kBlock) void int4_dequant_wide_kernel(
    const uint8_t* __restrict__ pool, const int32_t* __restrict__ slots,
    uint16_t* __restrict__ out_key, uint16_t* __restrict__ out_value, Int4Geom g,
    int num_rows) {
    constexpr int D = 128;
    const int j = threadIdx.x & 15;
    const int row = blockIdx.x * (kBlock / 16) + (threadIdx.x >> 4);
    if (row >= num_rows) return;
    const int t = row / g.H, h = row - t * g.H;
    const int slot = slots[t];
    if (slot < 0) return;
    int page, tib;
    page_of(slot, g.block_size, page, tib);
    const size_t cell = (size_t)tib * g.H + h;
    const uint8_t* base = pool + (size_t)page * g.page_size;
    const uint32_t kw = reinterpret_cast<const uint32_t*>(base + g.kc_off + cell * g.code_bytes)[j];
    const uint32_t vw = reinterpret_cast<const uint32_t*>(base + g.vc_off + cell * g.code_bytes)[j];
    const float ks = h2f(ld_u16(base + g.ks_off + cell * g.scale_bytes));
    const float vs = h2f(ld_u16(base + g.vs_off + cell * g.scale_bytes));
    const auto decode = [](uint32_t w, float sc) {
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float a = (float)(int)__builtin_amdgcn_sbfe((int)w, 8 * q, 4);
            const float b = (float)(int)__builtin_amdgcn_sbfe((int)w, 8 * q + 4, 4);
            o[q] = f2h2(a * sc, b * sc);
        }
        return u32x4{o[0], o[1], o[2], o[3]};
    };
    const size_t off = (size_t)row * D + 8 * j;
    __builtin_nontemporal_store(decode(kw, ks), reinterpret_cast<u32x4*>(out_key + off));
    __builtin_nontemporal_store(decode(vw, vs), reinterpret_cast<u32x4*>(out_value + off));
}

// ---------------------------------------------------------------------------
// Dense fp16 page (tq_dense_kernels.cu): a copy of each (token, head) row of
// D halves between [N, H, D] and the page cell, one dword per thread.
// ---------------------------------------------------------------------------
template <bool STORE>
__global__ __launch_bounds__(kBlock) void dense_copy_kernel(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
    uint16_t* __restrict__ out_key, uint16_t* __restrict__ out_value,
    const int32_t* __restrict__ slots, uint8_t* __restrict__ pool, DenseGeom g,
    long long num_dwords) {
    const long long i = (long long)blockIdx.x * kBlock + threadIdx.x;
    if (i >= num_dwords) return;
    const int per_row = g.D / 2;
    const long long row = i / per_row;
    const int d2 = (int)(i - row * per_row);
    const int t = (int)(row / g.H), h = (int)(row - (long long)t * g.H);
    const int slot = slots[t];
    if (slot < 0) return;
    int page, tib;
    page_of(slot, g.block_size, page, tib);
    const size_t cell = ((size_t)tib * g.H + h) * (size_t)g.D * 2 + 4 * (size_t)d2;
    uint8_t* base = pool + (size_t)page * g.page_size;
    uint32_t* pk = reinterpret_cast<uint32_t*>(base + g.k_off + cell);
    uint32_t* pv = reinterpret_cast<uint32_t*>(base + g.v_off + cell);
    if (STORE) {
        *pk = reinterpret_cast<const uint32_t*>(key)[i];
        *pv = reinterpret_cast<const uint32_t*>(value)[i];
    } else {
        reinterpret_cast<uint32_t*>(out_key)[i] = *pk;
        reinterpret_cast<uint32_t*>(out_value)[i] = *pv;
    }
}

// ---------------------------------------------------------------------------
// GPU SDPA reference (tq_attention_ref_kernel.cu:24-112): per (query, head),
// logits = <q, k> * (1/sqrt(D)) into logit_scratch, max, sum of exp,
// softmax-weighted V sum, fp16.  A workgroup of 4 waves per (query, head);
// wave w takes tokens w, w + 4, ... in the logit and V passes.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void sdpa_ref_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, uint16_t* __restrict__ output,
    float* __restrict__ logits, int H, int num_kv_tokens, float inv) {
    constexpr int L = D / 2, kW = 4;
    __shared__ float red[kW];
    __shared__ float acc[kW][D];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, j = lane % L;
    const int row = blockIdx.x;  // q * H + h
    const int h = row % H;
    const int N = num_kv_tokens;
    const uint32_t qq = *reinterpret_cast<const uint32_t*>(query + (size_t)row * D + 2 * j);
    const float q0 = h2f(qq & 0xffff), q1 = h2f(qq >> 16);
    float* lg = logits + (size_t)row * N;

    float mx = kInitMax;
    for (int t = w; t < N; t += kW) {
        const uint32_t kk =
            *reinterpret_cast<const uint32_t*>(key + ((size_t)t * H + h) * D + 2 * j);
        const float logit = tree_pair<L>(q0 * h2f(kk & 0xffff), q1 * h2f(kk >> 16)) * inv;
        if (lane == 0) lg[t] = logit;
        mx = fmaxf(mx, logit);
    }
    if (lane == 0) red[w] = mx;
    __syncthreads();  // also orders the logit stores before the reads below
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();

    float s = 0.0f;
    for (int t = tid; t < N; t += 256) s += expf(lg[t] - mx);
    s = sum_lanes<64>(s);
    if (lane == 0) red[w] = s;
    __syncthreads();
    s = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv_sum = s > 0.0f ? 1.0f / s : 1.0f;

    float a0 = 0.0f, a1 = 0.0f;
    for (int t = w; t < N; t += kW) {
        const float wt = expf(lg[t] - mx) * inv_sum;
        const uint32_t vv =
            *reinterpret_cast<const uint32_t*>(value + ((size_t)t * H + h) * D + 2 * j);
        a0 += wt * h2f(vv & 0xffff);
        a1 += wt * h2f(vv >> 16);
    }
    if (lane < L) {
        acc[w][2 * j] = a0;
        acc[w][2 * j + 1] = a1;
    }
    __syncthreads();
    if (tid < L) {
        const float o0 = (acc[0][2 * tid] + acc[1][2 * tid]) + (acc[2][2 * tid] + acc[3][2 * tid]);
        const float o1 = (acc[0][2 * tid + 1] + acc[1][2 * tid + 1]) +
                         (acc[2][2 * tid + 1] + acc[3][2 * tid + 1]);
        *reinterpret_cast<uint32_t*>(output + (size_t)row * D + 2 * tid) = f2h2(o0, o1);
    }
}

}  // namespace

#define TQ_DISPATCH_D(D_, ...)                                                   \
    switch (D_) {                                                                \
        case 2: { constexpr int kD = 2; __VA_ARGS__; } break;                    \
        case 4: { constexpr int kD = 4; __VA_ARGS__; } break;                    \
        case 8: { constexpr int kD = 8; __VA_ARGS__; } break;                    \
        case 16: { constexpr int kD = 16; __VA_ARGS__; } break;                  \
        case 32: { constexpr int kD = 32; __VA_ARGS__; } break;                  \
        case 64: { constexpr int kD = 64; __VA_ARGS__; } break;                  \
        case 128: { constexpr int kD = 128; __VA_ARGS__; } break;                \
        default: throw Error("head_dim must be a power of two in [2, 128]");     \
    }

static unsigned row_blocks(long long rows, int D) {
    const int rows_per_block = kBlock / (D / 2);
    return (unsigned)((rows + rows_per_block - 1) / rows_per_block);
}

void launch_qjl_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                     uint8_t* pool, const QjlGeom& g, int num_tokens, hipStream_t stream) {
    if (launch_qjl_wide_pack(key, value, slots, pool, g, num_tokens, stream)) return;
    const long long rows = (long long)num_tokens * g.H;
    if (rows <= 0) return;
    const float inv = inv_sqrt_d(g.D);
    TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(qjl_pack_kernel<kD>, dim3(row_blocks(rows, kD)),
                                          dim3(kBlock), 0, stream, key, value, slots, pool, g,
                                          (int)rows, inv));
    check_launch("qjl_pack_kv_kernel");
}

void launch_qjl_dequant(const uint8_t* pool, const int32_t* slots, uint16_t* out_key,
                        uint16_t* out_value, const QjlGeom& g, int num_tokens,
                        hipStream_t stream) {
    const long long rows = (long long)num_tokens * g.H;
    if (rows <= 0) return;
    if (launch_qjl_stream_dequant(pool, slots, out_key, out_value, g, num_tokens, stream)) return;
    const float inv = inv_sqrt_d(g.D);
    TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(qjl_dequant_kernel<kD>, dim3(row_blocks(rows, kD)),
                                          dim3(kBlock), 0, stream, pool, slots, out_key,
                                          out_value, g, (int)rows, inv));
    check_launch("qjl_dequant_kv_kernel");
}

void launch_qjl_attention(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                          uint16_t* output, const QjlGeom& g, int num_queries, int num_kv_tokens,
                          hipStream_t stream) {
    const int rows = num_queries * g.H;
    if (rows <= 0) return;
    if (launch_qjl_mfma_attention(query, pool, slots, output, g, num_queries, num_kv_tokens,
                                  stream))
        return;
    const float inv = inv_sqrt_d(g.D);
    // Enough waves to cover the chip several times, at least 32 tokens each.
    int splits = (2048 + rows - 1) / rows;
    splits = std::min(splits, std::max(1, (num_kv_tokens + 31) / 32));
    splits = std::max(splits, 1);
    const int tps = num_kv_tokens > 0 ? (num_kv_tokens + splits - 1) / splits : 0;
    if (tps > 0) splits = (num_kv_tokens + tps - 1) / tps;
    float* ws = static_cast<float*>(
        workspace(stream, (size_t)splits * rows * (g.D + 2) * sizeof(float)));
    TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(qjl_attn_partial_kernel<kD>, dim3(splits * rows),
                                          dim3(64), 0, stream, query, pool, slots, ws, g, rows,
                                          num_kv_tokens, tps, splits, inv));
    check_launch("qjl_fused_attn_partial");
    TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(qjl_attn_combine_kernel<kD>, dim3(rows), dim3(64), 0,
                                          stream, ws, output, rows, splits, inv));
    check_launch("qjl_fused_attn_combine");
}

void launch_int4_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                      uint8_t* pool, const Int4Geom& g, int num_tokens, hipStream_t stream) {
    const long long rows = (long long)num_tokens * g.H;
    if (rows <= 0) return;
    const auto al = [](uint64_t v, uint64_t a) { return (v & (a - 1)) == 0; };
    if (g.D == 128 && g.code_bytes == 64 && al(g.page_size, 4) && al(g.kc_off, 4) &&
        al(g.vc_off, 4) && al(reinterpret_cast<uintptr_t>(pool), 4) &&
        al(reinterpret_cast<uintptr_t>(key), 16) && al(reinterpret_cast<uintptr_t>(value), 16)) {
        hipLaunchKernelGGL(int4_pack_wide_kernel, dim3((unsigned)((rows + 15) / 16)),
                           dim3(kBlock), 0, stream, key, value, slots, pool, g, (int)rows);
        check_launch("tq_pack_kv_kernel");
        return;
    }
    TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(int4_pack_kernel<kD>, dim3(row_blocks(rows, kD)),
                                          dim3(kBlock), 0, stream, key, value, slots, pool, g,
                                          (int)rows));
    check_launch("tq_pack_kv_kernel");
}

void launch_int4_dequant(const uint8_t* pool, const int32_t* slots, uint16_t* out_key,
                         uint16_t* out_value, const Int4Geom& g, int num_tokens,
                         hipStream_t stream) {
    const long long rows = (long long)num_tokens * g.H;
    if (rows <= 0) return;
    const auto al = [](uint64_t v, uint64_t a) { return (v & (a - 1)) == 0; };
    if (g.D == 128 && g.code_bytes == 64 && al(g.page_size, 4) && al(g.kc_off, 4) &&
        al(g.vc_off, 4) && al(reinterpret_cast<uintptr_t>(pool), 4) &&
        al(reinterpret_cast<uintptr_t>(out_key), 16) && al(reinterpret_cast<uintptr_t>(out_value), 16)) {
        hipLaunchKernelGGL(int4_dequant_wide_kernel, dim3((unsigned)((rows + 15) / 16)),
                           dim3(kBlock), 0, stream, pool, slots, out_key, out_value, g, (int)rows);
        check_launch("tq_dequant_kv_kernel");
        return;
    }
    TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(int4_dequant_kernel<kD>, dim3(row_blocks(rows, kD)),
                                          dim3(kBlock), 0, stream, pool, slots, out_key,
                                          out_value, g, (int)rows));
    check_launch("tq_dequant_kv_kernel");
}

void launch_dense_copy(bool store, const uint16_t* key, const uint16_t* value, uint16_t* out_key,
                       uint16_t* out_value, const int32_t* slots, uint8_t* pool,
                       const DenseGeom& g, int num_tokens, hipStream_t stream) {
    const long long dwords = (long long)num_tokens * g.H * (g.D / 2);
    if (dwords <= 0) return;
    const unsigned blocks = (unsigned)((dwords + kBlock - 1) / kBlock);
    if (store)
        hipLaunchKernelGGL(dense_copy_kernel<true>, dim3(blocks), dim3(kBlock), 0, stream, key,
                           value, nullptr, nullptr, slots, pool, g, dwords);
    else
        hipLaunchKernelGGL(dense_copy_kernel<false>, dim3(blocks), dim3(kBlock), 0, stream,
                           nullptr, nullptr, out_key, out_value, slots, pool, g, dwords);
    check_launch(store ? "dense_store_kv_kernel" : "dense_load_kv_kernel");
}

void launch_attention_ref(const uint16_t* query, const uint16_t* key, const uint16_t* value,
                          uint16_t* output, float* logits, int H, int D, int num_queries,
                          int num_kv_tokens, hipStream_t stream) {
    const int rows = num_queries * H;
    if (rows <= 0) return;
    const float inv = inv_sqrt_d(D);
    TQ_DISPATCH_D(D, hipLaunchKernelGGL(sdpa_ref_kernel<kD>, dim3(rows), dim3(256), 0, stream,
                                        query, key, value, output, logits, H, num_kv_tokens,
                                        inv));
    check_launch("attention_ref_kernel");
}

}  // namespace tq

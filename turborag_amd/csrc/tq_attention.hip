// tq_attention.hip — fused decode attention over compressed pages (turbo_prod
// and turbo_mse) and the turbo_prod logits entry, gfx950.
//
// The reference runs one workgroup per (query row, kv head) that walks every
// token serially (src/cuda/tq_turbo_prod_kernels.cu:439-571,
// src/cuda/tq_turbo_mse_kernels.cu:302-417): 16 workgroups for a GQA 16/2
// decode step.  Here the token range is split (flash-decoding): each wave
// owns one (split, query row, kv head), keeps the reference's online softmax
// over its tokens in the rotated domain, and writes (m, l, acc[D]) partials;
// a combine kernel merges the splits with the usual log-sum-exp rescaling,
// normalises, applies the inverse WHT and the sign flip, and writes fp16.
// Logits follow the reference's convention <q, k> / sqrt(D) (:426, :531,
// turbo_mse :378).
#include <algorithm>

#include "tq_device.h"

namespace tq {
namespace {

using namespace dev;

constexpr float kInitMax = -1e30f;  // kInitMaxLogit, include/tq_shared_device.cuh:10

// Rotated query pair for lane j: qrot = WHT(q * s) * inv (:472-478).
template <int L>
__device__ __forceinline__ void rotate_query(const uint16_t* q, int h, int j, float inv,
                                             float& q0, float& q1) {
    const uint32_t qq = *reinterpret_cast<const uint32_t*>(q + 2 * j);
    const float sh = (h & 1) ? -1.0f : 1.0f;
    q0 = h2f(qq & 0xffff) * sh;
    q1 = h2f(qq >> 16) * (-sh);
    wht_pair<L>(q0, q1, j);
    q0 *= inv;
    q1 *= inv;
}

struct CellPtrs {
    const uint8_t* base;
    size_t cell;
};

__device__ __forceinline__ CellPtrs cell_of(const uint8_t* pool, const int32_t* slots, int t,
                                            int h, const PageGeom& g) {
    int page, tib;
    split_slot(slots[t], g, page, tib);
    return {pool + (size_t)page * g.page_size, (size_t)(tib * g.H + h)};
}

// ---------------------------------------------------------------------------
// Split-K partial: one wave per (split, row = q*H + h).
// ws[(split * rows + row) * (D + 2) + ...] = acc[0..D), m, l.
// ---------------------------------------------------------------------------
template <int D, bool PROD>
__global__ __launch_bounds__(64) void attn_partial_kernel(
    const uint16_t* __restrict__ query, const uint8_t* __restrict__ pool,
    const int32_t* __restrict__ slots, float* __restrict__ ws, PageGeom g, int rows,
    int num_kv_tokens, int tokens_per_split, int num_splits, float inv) {
    constexpr int L = D / 2;
    __shared__ float tk[16], tv[16];
    const int lane = threadIdx.x;
    if (lane < 16) {
        tk[lane] = PROD ? kK3[lane & 7] : kV4[lane];
        tv[lane] = kV4[lane];
    }
    __syncthreads();
    const int j = lane % L;
    const int split = blockIdx.x % num_splits;
    const int row = blockIdx.x / num_splits;
    const int h = row % g.H;

    float q0, q1;
    rotate_query<L>(query + (size_t)row * D, h, j, inv, q0, q1);

    const int t0 = split * tokens_per_split;
    const int t1 = min(num_kv_tokens, t0 + tokens_per_split);
    float m = kInitMax, l = 0.0f, a0 = 0.0f, a1 = 0.0f;
    for (int t = t0; t < t1; ++t) {
        const CellPtrs c = cell_of(pool, slots, t, h, g);
        const uint32_t kb = c.base[g.kc_off + c.cell * g.code_stride + j];
        const float ks = h2f(ld_u16(c.base + g.ks_off + c.cell * g.scale_stride));
        const uint32_t n0 = kb & 0xf, n1 = kb >> 4;
        float logit;
        if (PROD) {
            const float re = h2f(ld_u16(c.base + g.kres_off + c.cell * g.scale_stride));
            float s1 = q0 * tk[n0] + q1 * tk[n1];
            float s2 = ((n0 & 8) ? q0 : -q0) + ((n1 & 8) ? q1 : -q1);
            s1 = sum_lanes<L>(s1);
            s2 = sum_lanes<L>(s2);
            logit = (s1 + s2 * re) * ks * inv;
        } else {
            const float s1 = sum_lanes<L>(q0 * tk[n0] + q1 * tk[n1]);
            logit = s1 * ks * inv;
        }
        const float m_new = fmaxf(m, logit);
        const float a = expf(m - m_new), b = expf(logit - m_new);
        l = l * a + b;
        m = m_new;
        const uint32_t vb = c.base[g.vc_off + c.cell * g.code_stride + j];
        const float vs = h2f(ld_u16(c.base + g.vs_off + c.cell * g.scale_stride));
        a0 = a0 * a + b * (tv[vb & 0xf] * vs);
        a1 = a1 * a + b * (tv[vb >> 4] * vs);
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

// Merge splits, normalise, inverse WHT, sign flip, fp16 (:560-570).
template <int D>
__global__ __launch_bounds__(64) void attn_combine_kernel(const float* __restrict__ ws,
                                                          uint16_t* __restrict__ output,
                                                          PageGeom g, int rows, int num_splits,
                                                          float inv) {
    constexpr int L = D / 2;
    const int lane = threadIdx.x;
    const int j = lane % L;
    const int row = blockIdx.x;
    const int h = row % g.H;
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
    const float s0 = (h & 1) ? -inv : inv;
    const uint32_t o = (uint32_t)f2h(a0 * s0) | ((uint32_t)f2h(a1 * -s0) << 16);
    *reinterpret_cast<uint32_t*>(output + (size_t)row * D + 2 * j) = o;
}

// ---------------------------------------------------------------------------
// turbo_prod logits (:346-434): one thread per kv token, the rotated query of
// the workgroup's row in LDS.  blockIdx.x = row * tiles + tile.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void prod_logits_kernel(
    const uint16_t* __restrict__ query, const uint8_t* __restrict__ pool,
    const int32_t* __restrict__ slots, float* __restrict__ logits, PageGeom g, int num_kv_tokens,
    int tiles, float inv) {
    constexpr int L = D / 2;
    __shared__ float qs[D];
    __shared__ float tk[8];
    const int row = blockIdx.x / tiles, tile = blockIdx.x % tiles;
    const int h = row % g.H;
    if (threadIdx.x < 8) tk[threadIdx.x] = kK3[threadIdx.x];
    if (threadIdx.x < 64) {
        const int j = threadIdx.x % L;
        float q0, q1;
        rotate_query<L>(query + (size_t)row * D, h, j, inv, q0, q1);
        if (threadIdx.x < L) {
            qs[2 * j] = q0;
            qs[2 * j + 1] = q1;
        }
    }
    __syncthreads();
    const int t = tile * 256 + threadIdx.x;
    if (t >= num_kv_tokens) return;
    const CellPtrs c = cell_of(pool, slots, t, h, g);
    const uint8_t* kc = c.base + g.kc_off + c.cell * g.code_stride;
    const float ks = h2f(ld_u16(c.base + g.ks_off + c.cell * g.scale_stride));
    const float re = h2f(ld_u16(c.base + g.kres_off + c.cell * g.scale_stride));
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll 4
    for (int b = 0; b < D / 2; ++b) {
        const uint32_t kb = kc[b];
        const uint32_t n0 = kb & 0xf, n1 = kb >> 4;
        const float x0 = qs[2 * b], x1 = qs[2 * b + 1];
        s1 = fmaf(x0, tk[n0 & 7], s1);
        s1 = fmaf(x1, tk[n1 & 7], s1);
        s2 += ((n0 & 8) ? x0 : -x0) + ((n1 & 8) ? x1 : -x1);
    }
    logits[(size_t)row * num_kv_tokens + t] = (s1 * ks + s2 * (ks * re)) * inv;
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

void launch_attention(Scheme s, const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                      uint16_t* output, const PageGeom& g, int num_queries, int num_kv_tokens,
                      hipStream_t stream) {
    const int rows = num_queries * g.H;
    if (rows <= 0) return;
    // Enough waves to cover the chip several times, at least 32 tokens each.
    int splits = (2048 + rows - 1) / rows;
    splits = std::min(splits, std::max(1, (num_kv_tokens + 31) / 32));
    splits = std::max(splits, 1);
    const int tps = num_kv_tokens > 0 ? (num_kv_tokens + splits - 1) / splits : 0;
    if (tps > 0) splits = (num_kv_tokens + tps - 1) / tps;
    const size_t ws_bytes = (size_t)splits * rows * (g.D + 2) * sizeof(float);
    float* ws = static_cast<float*>(workspace(stream, ws_bytes));
    const float inv = inv_sqrt_d(g.D);
    const bool prod = s == Scheme::Prod;
    if (prod) {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL((attn_partial_kernel<kD, true>),
                                              dim3(splits * rows), dim3(64), 0, stream, query,
                                              pool, slots, ws, g, rows, num_kv_tokens, tps,
                                              splits, inv));
    } else {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL((attn_partial_kernel<kD, false>),
                                              dim3(splits * rows), dim3(64), 0, stream, query,
                                              pool, slots, ws, g, rows, num_kv_tokens, tps,
                                              splits, inv));
    }
    check_launch(prod ? "turbo_prod_fused_attn_partial" : "turbo_mse_fused_attn_partial");
    TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(attn_combine_kernel<kD>, dim3(rows), dim3(64), 0,
                                          stream, ws, output, g, rows, splits, inv));
    check_launch(prod ? "turbo_prod_fused_attn_combine" : "turbo_mse_fused_attn_combine");
}

void launch_logits(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                   float* logits, const PageGeom& g, int num_queries, int num_kv_tokens,
                   hipStream_t stream) {
    const int rows = num_queries * g.H;
    if (rows <= 0 || num_kv_tokens <= 0) return;
    const int tiles = (num_kv_tokens + 255) / 256;
    const float inv = inv_sqrt_d(g.D);
    TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(prod_logits_kernel<kD>, dim3(rows * tiles), dim3(256),
                                          0, stream, query, pool, slots, logits, g,
                                          num_kv_tokens, tiles, inv));
    check_launch("turbo_prod_fused_attention_logits_kernel");
}

}  // namespace tq

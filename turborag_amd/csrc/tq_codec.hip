// tq_codec.hip — turbo_prod and turbo_mse pack / dequant kernels for gfx950.
//
// Mapping: a row (one token-head, D values) is owned by D/2 lanes of a wave64,
// two elements per lane (see tq_device.h); a 256-thread workgroup covers
// 512/D rows, rows ordered token-major like the [N, H, D] tensors, so global
// loads and stores of a wave are contiguous.  The WHT and the RMS trees are
// register/xor-shuffle butterflies that repeat the reference's float
// operation order, so codes, scales and dequantized halves are bit-identical
// to the reference's CUDA kernels (given correctly rounded / and sqrt, which
// this library is compiled for).
#include "tq_device.h"

namespace tq {
namespace {

using namespace dev;

constexpr int kBlock = 256;

// ---------------------------------------------------------------------------
// turbo_prod pack — src/cuda/tq_turbo_prod_kernels.cu:110-260
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(kBlock) void prod_pack_kernel(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
    const int32_t* __restrict__ slots, uint8_t* __restrict__ pool, PageGeom g, int num_rows,
    float inv) {
    constexpr int L = D / 2;
    const int j = threadIdx.x % L;
    const int row = blockIdx.x * (kBlock / L) + threadIdx.x / L;
    const bool valid = row < num_rows;
    const int rr = valid ? row : num_rows - 1;
    const int t = rr / g.H, h = rr % g.H;

    const size_t off = (size_t)rr * D + 2 * j;
    const uint32_t kk = *reinterpret_cast<const uint32_t*>(key + off);
    const uint32_t vv = *reinterpret_cast<const uint32_t*>(value + off);
    // s(2j, h) = (-1)^h, s(2j+1, h) = -(-1)^h; multiplication by +-1 is exact.
    const float sh = (h & 1) ? -1.0f : 1.0f;
    float k0 = h2f(kk & 0xffff) * sh, k1 = h2f(kk >> 16) * (-sh);
    float v0 = h2f(vv & 0xffff) * sh, v1 = h2f(vv >> 16) * (-sh);

    wht_pair<L>(k0, k1, j);
    wht_pair<L>(v0, v1, j);
    k0 *= inv; k1 *= inv; v0 *= inv; v1 *= inv;

    float krms = sqrtf(tree_pair<L>(k0 * k0, k1 * k1) / (float)D);
    if (krms < kMinRMS) krms = kMinRMS;
    float vrms = sqrtf(tree_pair<L>(v0 * v0, v1 * v1) / (float)D);
    if (vrms < kMinRMS) vrms = kMinRMS;

    const float kn0 = clamp_ref(k0 / krms, -2.5f, 2.5f), kn1 = clamp_ref(k1 / krms, -2.5f, 2.5f);
    const float vn0 = clamp_ref(v0 / vrms, -2.75f, 2.75f), vn1 = clamp_ref(v1 / vrms, -2.75f, 2.75f);
    float lv0, lv1;
    const int c0 = nearest_k3(kn0, lv0), c1 = nearest_k3(kn1, lv1);
    const float e0 = kn0 - lv0, e1 = kn1 - lv1;
    float rms_e = sqrtf(tree_pair<L>(e0 * e0, e1 * e1) / (float)D);
    if (rms_e < kMinRMS) rms_e = kMinRMS;
    const int q0 = nearest_v4(vn0), q1 = nearest_v4(vn1);

    if (!valid) return;
    const int slot = slots[t];
    if (slot < 0) return;
    int page, tib;
    split_slot(slot, g, page, tib);
    const int cell = tib * g.H + h;
    uint8_t* base = pool + (size_t)page * g.page_size;
    const uint32_t n0 = (e0 >= 0.0f ? 8u : 0u) | (uint32_t)c0;
    const uint32_t n1 = (e1 >= 0.0f ? 8u : 0u) | (uint32_t)c1;
    base[g.kc_off + (size_t)cell * g.code_stride + j] = (uint8_t)(n0 | (n1 << 4));
    base[g.vc_off + (size_t)cell * g.code_stride + j] = (uint8_t)(q0 | (q1 << 4));
    if (j == 0) {
        *reinterpret_cast<uint16_t*>(base + g.ks_off + (size_t)cell * g.scale_stride) = f2h(krms);
        *reinterpret_cast<uint16_t*>(base + g.kres_off + (size_t)cell * g.scale_stride) = f2h(rms_e);
        *reinterpret_cast<uint16_t*>(base + g.vs_off + (size_t)cell * g.scale_stride) = f2h(vrms);
    }
}

// ---------------------------------------------------------------------------
// turbo_mse pack — src/cuda/tq_turbo_mse_kernels.cu:65-136, 186-237.
// The pair sum red[t] = x0*x0 + x1*x1 (:108) is evaluated as
// fmaf(x0, x0, x1*x1), the contraction nvcc applies at its default -fmad=true.
// ---------------------------------------------------------------------------
template <int L>
__device__ __forceinline__ uint32_t mse_quantize_pair(float x0, float x1, int j, float inv,
                                                      float D, float& rms) {
    wht_pair<L>(x0, x1, j);
    x0 *= inv;
    x1 *= inv;
    rms = sqrtf(tree_one<L>(fmaf(x0, x0, x1 * x1)) / D);
    if (rms < kMinRMS) rms = kMinRMS;
    const int qa = nearest_v4(clamp_ref(x0 / rms, -2.75f, 2.75f));
    const int qb = nearest_v4(clamp_ref(x1 / rms, -2.75f, 2.75f));
    return (uint32_t)((qb << 4) | qa);
}

template <int D>
__global__ __launch_bounds__(kBlock) void mse_pack_kernel(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
    const int32_t* __restrict__ slots, uint8_t* __restrict__ pool, PageGeom g, int num_rows,
    float inv) {
    constexpr int L = D / 2;
    const int j = threadIdx.x % L;
    const int row = blockIdx.x * (kBlock / L) + threadIdx.x / L;
    const bool valid = row < num_rows;
    const int rr = valid ? row : num_rows - 1;
    const int t = rr / g.H, h = rr % g.H;
    const size_t off = (size_t)rr * D + 2 * j;
    const uint32_t kk = *reinterpret_cast<const uint32_t*>(key + off);
    const uint32_t vv = *reinterpret_cast<const uint32_t*>(value + off);
    const float sh = (h & 1) ? -1.0f : 1.0f;
    float krms, vrms;
    const uint32_t kb = mse_quantize_pair<L>(h2f(kk & 0xffff) * sh, h2f(kk >> 16) * (-sh), j, inv,
                                             (float)D, krms);
    const uint32_t vb = mse_quantize_pair<L>(h2f(vv & 0xffff) * sh, h2f(vv >> 16) * (-sh), j, inv,
                                             (float)D, vrms);
    if (!valid) return;
    const int slot = slots[t];
    if (slot < 0) return;
    int page, tib;
    split_slot(slot, g, page, tib);
    const int cell = tib * g.H + h;
    uint8_t* base = pool + (size_t)page * g.page_size;
    base[g.kc_off + (size_t)cell * g.code_stride + j] = (uint8_t)kb;
    base[g.vc_off + (size_t)cell * g.code_stride + j] = (uint8_t)vb;
    if (j == 0) {
        *reinterpret_cast<uint16_t*>(base + g.ks_off + (size_t)cell * g.scale_stride) = f2h(krms);
        *reinterpret_cast<uint16_t*>(base + g.vs_off + (size_t)cell * g.scale_stride) = f2h(vrms);
    }
}

// ---------------------------------------------------------------------------
// Dequant — turbo_prod :265-341, turbo_mse :138-184 / :239-287.
// prod K: (K3[n&7] + re*(n&8 ? 1 : -1)) * ks;  V and turbo_mse: V4[n] * rms.
// Then WHT and out = fp16((y * inv) * s_i) (written as y * (s_i*inv): equal,
// since negation commutes with rounding).
// ---------------------------------------------------------------------------
template <int D, bool PROD>
__global__ __launch_bounds__(kBlock) void dequant_kernel(
    const uint8_t* __restrict__ pool, const int32_t* __restrict__ slots,
    uint16_t* __restrict__ out_key, uint16_t* __restrict__ out_value, PageGeom g, int num_rows,
    float inv) {
    constexpr int L = D / 2;
    __shared__ float tk[16], tv[16];
    if (threadIdx.x < 16) {
        tk[threadIdx.x] = PROD ? kK3[threadIdx.x & 7] : kV4[threadIdx.x];
        tv[threadIdx.x] = kV4[threadIdx.x];
    }
    __syncthreads();

    const int j = threadIdx.x % L;
    const int row = blockIdx.x * (kBlock / L) + threadIdx.x / L;
    const bool valid = row < num_rows;
    const int rr = valid ? row : num_rows - 1;
    const int t = rr / g.H, h = rr % g.H;
    const int slot = slots[t];
    const bool live = valid && slot >= 0;
    float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
    if (slot >= 0) {
        int page, tib;
        split_slot(slot, g, page, tib);
        const int cell = tib * g.H + h;
        const uint8_t* base = pool + (size_t)page * g.page_size;
        const uint32_t kb = base[g.kc_off + (size_t)cell * g.code_stride + j];
        const uint32_t vb = base[g.vc_off + (size_t)cell * g.code_stride + j];
        const float ks = h2f(ld_u16(base + g.ks_off + (size_t)cell * g.scale_stride));
        const float vs = h2f(ld_u16(base + g.vs_off + (size_t)cell * g.scale_stride));
        const uint32_t n0 = kb & 0xf, n1 = kb >> 4;
        if (PROD) {
            const float re = h2f(ld_u16(base + g.kres_off + (size_t)cell * g.scale_stride));
            k0 = (tk[n0] + re * ((n0 & 8) ? 1.0f : -1.0f)) * ks;
            k1 = (tk[n1] + re * ((n1 & 8) ? 1.0f : -1.0f)) * ks;
        } else {
            k0 = tk[n0] * ks;
            k1 = tk[n1] * ks;
        }
        v0 = tv[vb & 0xf] * vs;
        v1 = tv[vb >> 4] * vs;
    }
    wht_pair<L>(k0, k1, j);
    wht_pair<L>(v0, v1, j);
    if (!live) return;
    const float s0 = (h & 1) ? -inv : inv;  // s(2j, h) * inv; s(2j+1, h) = -s(2j, h)
    const uint32_t ko = (uint32_t)f2h(k0 * s0) | ((uint32_t)f2h(k1 * -s0) << 16);
    const uint32_t vo = (uint32_t)f2h(v0 * s0) | ((uint32_t)f2h(v1 * -s0) << 16);
    const size_t off = (size_t)rr * D + 2 * j;
    *reinterpret_cast<uint32_t*>(out_key + off) = ko;
    *reinterpret_cast<uint32_t*>(out_value + off) = vo;
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
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

void launch_pack(Scheme s, const uint16_t* key, const uint16_t* value, const int32_t* slots,
                 uint8_t* pool, const PageGeom& g, int num_tokens, hipStream_t stream) {
    const int rows = num_tokens * g.H;
    if (rows <= 0) return;
    const int rpb = kBlock / (g.D / 2);
    const dim3 grid((rows + rpb - 1) / rpb);
    const float inv = inv_sqrt_d(g.D);
    if (s == Scheme::Prod) {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(prod_pack_kernel<kD>, grid, dim3(kBlock), 0, stream,
                                              key, value, slots, pool, g, rows, inv));
        check_launch("turbo_prod_pack_kv_kernel");
    } else {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(mse_pack_kernel<kD>, grid, dim3(kBlock), 0, stream,
                                              key, value, slots, pool, g, rows, inv));
        check_launch("turbo_mse_pack_kv_kernel");
    }
}

void launch_dequant(Scheme s, const uint8_t* pool, const int32_t* slots, uint16_t* out_key,
                    uint16_t* out_value, const PageGeom& g, int num_tokens, hipStream_t stream) {
    const int rows = num_tokens * g.H;
    if (rows <= 0) return;
    const int rpb = kBlock / (g.D / 2);
    const dim3 grid((rows + rpb - 1) / rpb);
    const float inv = inv_sqrt_d(g.D);
    if (s == Scheme::Prod) {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL((dequant_kernel<kD, true>), grid, dim3(kBlock), 0,
                                              stream, pool, slots, out_key, out_value, g, rows,
                                              inv));
        check_launch("turbo_prod_dequant_kv_kernel");
    } else {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL((dequant_kernel<kD, false>), grid, dim3(kBlock), 0,
                                              stream, pool, slots, out_key, out_value, g, rows,
                                              inv));
        check_launch("turbo_mse_dequant_kv_kernel");
    }
}

}  // namespace tq

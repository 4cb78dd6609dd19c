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
#include <algorithm>

#include "tq_device.h"

namespace tq {
namespace {

using namespace dev;

constexpr int kBlock = 256;
// Lanes per row of the wide pack: 8 rows per wave share every per-row
// instruction (RMS, reciprocal, square roots); 16 lanes ran 15% slower, and
// 4 lanes (200 VGPRs, two waves per SIMD) 43% slower.
constexpr int kPackLanes = 8;

// ---------------------------------------------------------------------------
// turbo_prod pack — src/cuda/tq_turbo_prod_kernels.cu:110-260
// ---------------------------------------------------------------------------
// dbg: the reference kernel's debug buffers (:216-217, :243-246), written
// for every row when non-null (they depend on K/V only, not on the slot).
template <int D>
__global__ __launch_bounds__(kBlock) void prod_pack_kernel(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
    const int32_t* __restrict__ slots, uint8_t* __restrict__ pool, PageGeom g, int num_rows,
    float inv, PackDebug dbg) {
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
    if (dbg.k_rot) *reinterpret_cast<float2*>(dbg.k_rot + off) = make_float2(k0, k1);
    if (dbg.v_rot) *reinterpret_cast<float2*>(dbg.v_rot + off) = make_float2(v0, v1);
    if (dbg.kn) *reinterpret_cast<float2*>(dbg.kn + off) = make_float2(kn0, kn1);
    if (dbg.vn) *reinterpret_cast<float2*>(dbg.vn + off) = make_float2(vn0, vn1);
    if (dbg.kidx) *reinterpret_cast<int2*>(dbg.kidx + off) = make_int2(c0, c1);
    if (dbg.vidx) *reinterpret_cast<int2*>(dbg.vidx + off) = make_int2(q0, q1);
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
// Pack, wide form (D = 64, 128): R lanes per (token, head) row, 64/R rows
// per wave.  Lane j owns the element pairs (2Rc + 2j, 2Rc + 2j + 1) of the
// C = D/2R chunks c, in registers k = 2c and 2c + 1.  The reference's
// butterfly stage len pairs elements i and i + len: in-lane for len = 1 and
// len >= 2R (chunks c and c ^ (len/2R)), lanes j and j ^ (len/2) for
// len = 2 .. R.  Its halving trees (r[i] += r[i + s], s = n/2 .. 1) run
// in-lane over chunks first (s >= 2R), then across lanes (s = R .. 2, one or
// two values per lane), and end in-lane (s = 1): most of the adds stay in
// registers.  Operation order per element is the reference's, so codes and
// scales are bit-identical to the one-row-per-wave form above.  Code byte
// Rc + j of a cell is the lane's chunk c.
// ---------------------------------------------------------------------------
// Lane order of a pack row: physical lane p (of 8) holds logical lane
// j = p for p < 4 and j = p ^ 3 for p >= 4.  Then logical j ^ 1 and j ^ 2
// are physical p ^ 1 and p ^ 2 (quad_perm), and logical j ^ 4 is physical
// 7 - p (row_half_mirror): every partner exchange is one DPP operand.
__device__ __forceinline__ int pack_lane(int p) { return (p & 4) ? p ^ 3 : p; }

template <int M>
__device__ __forceinline__ float row8_xor(float v) {
    constexpr int ctrl = M == 1 ? 0xB1 : (M == 2 ? 0x4E : 0x141);
    static_assert(M == 1 || M == 2 || M == 4, "row of 8 lanes");
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, true));
}

// y[k] = y[k] + c * (partner's y[k]) for 8 values, the partner read by DPP
// (v_fmac_f32_dpp).  The s_nop gives the two wait states a DPP read needs
// after the VALU write of its source.
#define TQ_FMAC8(CTRL)                                                                     \
    "s_nop 1\n\t"                                                                          \
    "v_fmac_f32_dpp %0, %0, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                     \
    "v_fmac_f32_dpp %1, %1, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                     \
    "v_fmac_f32_dpp %2, %2, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                     \
    "v_fmac_f32_dpp %3, %3, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                     \
    "v_fmac_f32_dpp %4, %4, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                     \
    "v_fmac_f32_dpp %5, %5, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                     \
    "v_fmac_f32_dpp %6, %6, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                     \
    "v_fmac_f32_dpp %7, %7, %8 " CTRL " row_mask:0xf bank_mask:0xf"

template <int M>
__device__ __forceinline__ void fmac_partner8(float* y, float c) {
    if constexpr (M == 1)
        asm(TQ_FMAC8("quad_perm:[1,0,3,2]")
            : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]), "+v"(y[4]), "+v"(y[5]),
              "+v"(y[6]), "+v"(y[7])
            : "v"(c));
    else if constexpr (M == 2)
        asm(TQ_FMAC8("quad_perm:[2,3,0,1]")
            : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]), "+v"(y[4]), "+v"(y[5]),
              "+v"(y[6]), "+v"(y[7])
            : "v"(c));
    else
        asm(TQ_FMAC8("row_half_mirror")
            : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]), "+v"(y[4]), "+v"(y[5]),
              "+v"(y[6]), "+v"(y[7])
            : "v"(c));
}
#undef TQ_FMAC8

// Butterfly stages len = 2 .. 64 of a row held as chunks (len = 1 is done by
// the caller: it carries the sign flip).  The cross-lane stages len = 2, 4, 8
// pair logical lanes j and j ^ m (m = len/2): the lower lane needs
// x + partner, the upper partner - x.  Each lane instead keeps
// y = sigma_j * x and applies y += c * partner_y with c = +1 (lower) or -1
// (upper), one fused DPP op: both lanes of a pair carry the same sigma, so
// the lower gets sigma * (x + x'), the upper -sigma * (x' - x) exactly
// (fp32 rounding is symmetric in sign), and sigma flips on upper lanes.
// After the three stages sigma_j = (-1)^popcount(j); the caller folds it
// into the exact scale.  The in-lane chunk stages len = 16 .. 64 are linear,
// so sigma passes through them.
template <int C>
__device__ __forceinline__ void wht_chunks(float (&x)[2 * C], int j) {
    static_assert((2 * C) % 8 == 0, "blocks of 8 values");
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
        const float c = (j & m) ? -1.0f : 1.0f;
#pragma unroll
        for (int k = 0; k < 2 * C; k += 8) {
            if (m == 1) fmac_partner8<1>(x + k, c);
            else if (m == 2) fmac_partner8<2>(x + k, c);
            else fmac_partner8<4>(x + k, c);
        }
    }
    // len = 16 .. 64: chunks c and c + len/16.
#pragma unroll
    for (int d = 1; d < C; d <<= 1)
#pragma unroll
        for (int c = 0; c < C; ++c)
            if ((c & d) == 0)
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const float u = x[2 * c + b], w = x[2 * (c + d) + b];
                    x[2 * c + b] = u + w;
                    x[2 * (c + d) + b] = u - w;
                }
}

// Halving tree over the row's 16C values r[2c + b] (element 16c + 2j + b):
// s = 8C .. 16 in-lane over chunks, s = 8 .. 2 across logical lanes j ^ s/2,
// s = 1 in-lane.  Every lane ends with the total.
template <int C>
__device__ __forceinline__ float tree_chunks(float (&r)[2 * C]) {
#pragma unroll
    for (int d = C / 2; d >= 1; d >>= 1)
#pragma unroll
        for (int k = 0; k < 2 * d; ++k) r[k] += r[k + 2 * d];
    r[0] += row8_xor<4>(r[0]);
    r[1] += row8_xor<4>(r[1]);
    r[0] += row8_xor<2>(r[0]);
    r[1] += row8_xor<2>(r[1]);
    r[0] += row8_xor<1>(r[0]);
    r[1] += row8_xor<1>(r[1]);
    return r[0] + r[1];
}

// Halving tree over the row's 8C pair sums q[c] (pair 8c + j): s = 4C .. 8
// in-lane over chunks, s = 4 .. 1 across logical lanes.
template <int C>
__device__ __forceinline__ float tree_chunk_pairs(float (&q)[C]) {
#pragma unroll
    for (int d = C / 2; d >= 1; d >>= 1)
#pragma unroll
        for (int c = 0; c < d; ++c) q[c] += q[c + d];
    q[0] += row8_xor<4>(q[0]);
    q[0] += row8_xor<2>(q[0]);
    q[0] += row8_xor<1>(q[0]);
    return q[0];
}

// One tensor's row, held as chunks: rotation (the first stage from the fp16
// pairs), RMS, codes packed two per byte.  kCodesK3: 3-bit K code + residual
// sign and the residual RMS (turbo_prod K); kCodesV4: 4-bit code, RMS of the
// squares (turbo_prod V); kCodesV4Pairs: 4-bit code, RMS of the pair sums
// fmaf(x0, x0, x1 * x1) (turbo_mse, tq_turbo_mse_kernels.cu:108, contracted).
// kCodesSigns: the QJL-1b K sign bits (x / rms >= 0) of the element pair,
// two bits per chunk, and the RMS of the squares.
constexpr int kCodesK3 = 0, kCodesV4 = 1, kCodesV4Pairs = 2, kCodesSigns = 3;
template <int C, int MODE>
__device__ __forceinline__ void quantize_chunks(const uint32_t (&w)[C], int j, float sinv,
                                                const PackTables& tab, uint32_t (&bytes)[C],
                                                float& rms, float& rms_e) {
    constexpr int E = 2 * C, D = 16 * C;
    float x[E];
#pragma unroll
    for (int c = 0; c < C; ++c) half_pair_diff_sum(w[c], x[2 * c], x[2 * c + 1]);
    wht_chunks<C>(x, j);
#pragma unroll
    for (int k = 0; k < E; ++k) x[k] *= sinv;
    if constexpr (MODE == kCodesV4Pairs) {
        float q[C];
#pragma unroll
        for (int c = 0; c < C; ++c) q[c] = fmaf(x[2 * c], x[2 * c], x[2 * c + 1] * x[2 * c + 1]);
        rms = sqrtf(tree_chunk_pairs<C>(q) / (float)D);
    } else {
        float r[E];
#pragma unroll
        for (int k = 0; k < E; ++k) r[k] = x[k] * x[k];
        rms = sqrtf(tree_chunks<C>(r) / (float)D);
    }
    if (rms < kMinRMS) rms = kMinRMS;
    const float y = 1.0f / rms;
    uint32_t n4[E];
    if constexpr (MODE == kCodesK3) {
        float r[E];
#pragma unroll
        for (int k = 0; k < E; ++k) {
            // fmin/fmax clamp a NaN to the low bound, whose codes (0) are the
            // reference's for NaN; its residual is made NaN below.
            const float kn = fminf(fmaxf(div_by(x[k], rms, y), -2.5f), 2.5f);
            float level;
            n4[k] = k3_nibble(kn, tab, level);
            const float e = kn - level;
            r[k] = e * e;
        }
        rms_e = sqrtf(tree_chunks<C>(r) / (float)D);
        if (rms_e < kMinRMS) rms_e = kMinRMS;
        // The rotation spreads a non-finite input over the whole row: then
        // every K/rms is NaN, the reference's residual RMS is NaN, and the
        // codes above are its codes for NaN (index 0, sign 0).
        if (!(rms <= 3.402823466e38f)) rms_e = __builtin_nanf("");
    } else if constexpr (MODE == kCodesSigns) {
        // x / rms >= 0 is x >= 0 for a finite rms >= 1e-8 (no quotient of a
        // sum of fp16 values that is not zero underflows); a non-finite rms
        // means a non-finite row, every quotient NaN: bit 0.
        const bool fin = rms <= 3.402823466e38f;
#pragma unroll
        for (int c = 0; c < C; ++c)
            bytes[c] = (fin && x[2 * c] >= 0.0f ? 1u : 0u) | (fin && x[2 * c + 1] >= 0.0f ? 2u : 0u);
        return;
    } else {
#pragma unroll
        for (int k = 0; k < E; ++k) n4[k] = v4_code(div_by(x[k], rms, y), tab);
    }
#pragma unroll
    for (int c = 0; c < C; ++c) bytes[c] = n4[2 * c] | (n4[2 * c + 1] << 4);
}

// The K/V inputs and page pool of each layer of a pack launch (passed by
// value in the kernel arguments); every layer shares the slot mapping.
template <int ML>
struct PackSet {
    const uint16_t* key[ML];
    const uint16_t* value[ML];
    uint8_t* pool[ML];
};
constexpr int kMaxPackLayersPerLaunch = 64;

// SCH: 0 turbo_mse, 1 turbo_prod, 2 the reference's unexported QJL-1b page
// (tq_qjl_kernels.cu:72-181: K sign bits, V 4-bit codes, sign flip (-1)^i
// without the head term).  ML > 1: layer blockIdx.y of the set (one launch
// packs every layer of a document).
template <int D, int SCH, int ML = 1>
__global__ __launch_bounds__(kBlock) void pack_wide_kernel(const PackSet<ML> set,
                                                           const int32_t* __restrict__ slots,
                                                           PageGeom g, int num_rows, float inv) {
    const int layer = ML == 1 ? 0 : (int)blockIdx.y;
    const uint16_t* __restrict__ key = set.key[layer];
    const uint16_t* __restrict__ value = set.value[layer];
    uint8_t* __restrict__ pool = set.pool[layer];
    constexpr int R = kPackLanes, C = D / (2 * R);
    static_assert(C == 4 || C == 8, "D = 64 or 128");
    constexpr bool PROD = SCH == 1, QJL = SCH == 2;
    __shared__ PackTables tab;
    const int j = pack_lane(threadIdx.x & (R - 1));
    const int row = blockIdx.x * (kBlock / R) + threadIdx.x / R;
    const bool valid = row < num_rows;
    const int rr = valid ? row : num_rows - 1;
    const int t = g.h_shift >= 0 ? rr >> g.h_shift : rr / g.H;
    const int h = rr - t * g.H;
    const uint32_t* kr = reinterpret_cast<const uint32_t*>(key + (size_t)rr * D) + j;
    const uint32_t* vr = reinterpret_cast<const uint32_t*>(value + (size_t)rr * D) + j;
    // The table word, the row's K words and its slot go out together; the V
    // words right after the table is stored, so they arrive during the K
    // quantization (the compiler had issued the V words after it and the
    // slot just before the stores: per-layer launches 6.9 -> 6.6 us, one
    // launch for 36 layers 3.05 -> 2.94 us per layer, config 2 turbo_prod).
    const uint32_t tw = reinterpret_cast<const uint32_t*>(
        &kPackTables)[min((int)threadIdx.x, kPackTableWords - 1)];
    uint32_t kw[C], vw[C];
#pragma unroll
    for (int c = 0; c < C; ++c) kw[c] = kr[R * c];
    const int slot_raw = slots[t];
    __builtin_amdgcn_sched_barrier(0);
    if (threadIdx.x < kPackTableWords) reinterpret_cast<uint32_t*>(&tab)[threadIdx.x] = tw;
    __syncthreads();
#pragma unroll
    for (int c = 0; c < C; ++c) vw[c] = vr[R * c];
    __builtin_amdgcn_sched_barrier(0);
    // s(i, h) = (-1)^(i + h) = sh * (-1)^b for element i = 2Rc + 2j + b.  The
    // first butterfly stage on (sh*a, -sh*b) gives (sh*(a - b), sh*(a + b));
    // fp32 rounding is symmetric in sign, so every later value is sh times
    // the one computed without it (up to the sign of exact zeros, which no
    // code or scale sees).  sh and the lane sign of wht_chunks are folded
    // into the exact scale +-1/sqrt(D).
    const float sinv = (((QJL ? 0 : h) ^ __popc(j)) & 1) ? -inv : inv;
    // K, then V: one tensor's values live at a time.
    uint32_t kbyte[C], vbyte[C];
    float krms, vrms, rms_e = 0.0f, unused;
    quantize_chunks<C, QJL ? kCodesSigns : PROD ? kCodesK3 : kCodesV4Pairs>(kw, j, sinv, tab, kbyte,
                                                                           krms, rms_e);
    __builtin_amdgcn_sched_barrier(0);
    quantize_chunks<C, QJL || PROD ? kCodesV4 : kCodesV4Pairs>(vw, j, sinv, tab, vbyte, vrms,
                                                               unused);
    // QJL: the sign byte of elements 8b .. 8b + 7 gathers two bits from each
    // of four lanes (logical j ^ 1, j ^ 2: quad DPP); chunk c gives bytes 2c
    // (lanes 0-3) and 2c + 1 (lanes 4-7), bits 2(j % 4), 2(j % 4) + 1.
    uint32_t kbits[C / 4] = {};
    if constexpr (QJL) {
#pragma unroll
        for (int c = 0; c < C; ++c) kbits[c >> 2] |= kbyte[c] << (8 * (c & 3) + 2 * (j & 3));
#pragma unroll
        for (int q = 0; q < C / 4; ++q) {
            kbits[q] |= __float_as_uint(row8_xor<1>(__uint_as_float(kbits[q])));
            kbits[q] |= __float_as_uint(row8_xor<2>(__uint_as_float(kbits[q])));
        }
    }
    if (!valid) return;
    const int slot = slot_raw;
    if (slot < 0) return;
    int page, tib;
    split_slot(slot, g, page, tib);
    const size_t cell = (size_t)(tib * g.H + h);
    uint8_t* base = pool + (size_t)page * g.page_size;
    // Element pair (2b, 2b+1) is byte b (low nibble even): chunk c of lane j
    // is byte Rc + j.
    uint8_t* vc = base + g.vc_off + cell * g.code_stride + j;
    if constexpr (QJL) {
        if ((j & 3) == 0) {
            uint8_t* kb = base + g.kc_off + cell * (D / 8) + (j >> 2);
#pragma unroll
            for (int c = 0; c < C; ++c) kb[2 * c] = (uint8_t)(kbits[c >> 2] >> (8 * (c & 3)));
        }
    } else {
        uint8_t* kc = base + g.kc_off + cell * g.code_stride + j;
#pragma unroll
        for (int c = 0; c < C; ++c) kc[R * c] = (uint8_t)kbyte[c];
    }
#pragma unroll
    for (int c = 0; c < C; ++c) vc[R * c] = (uint8_t)vbyte[c];
    if (j == 0) {
        *reinterpret_cast<uint16_t*>(base + g.ks_off + cell * g.scale_stride) = f2h(krms);
        if (PROD)
            *reinterpret_cast<uint16_t*>(base + g.kres_off + cell * g.scale_stride) = f2h(rms_e);
        *reinterpret_cast<uint16_t*>(base + g.vs_off + cell * g.scale_stride) = f2h(vrms);
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
    float inv, OutLayout ol) {
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
    const size_t off = ol.offset(t, h) + 2 * j;
    // Plain stores: rows of fewer than 64 elements share 128-byte lines with
    // their neighbours, and non-temporal pieces of a line each go to memory.
    *reinterpret_cast<uint32_t*>(out_key + off) = ko;
    *reinterpret_cast<uint32_t*>(out_value + off) = vo;
}

// ---------------------------------------------------------------------------
// Dequant, streaming form (D = 32, 64, 128).  A row is owned by LPR = D/32
// lanes; lane j holds the four 8-element chunks j + LPR*m (m = 0..3), so WHT
// stages len = 1, 2, 4 and len >= 8*LPR are register butterflies and the
// stages in between cross lanes (quad DPP moves, VALU rate).  For D = 128
// the output leaves as non-temporal stores of whole 128-byte lines (two rows
// trade chunks first); for D = 32, 64 store m of the row's lanes writes
// 16*LPR contiguous bytes with plain stores, which the L2 merges into lines
// (non-temporal pieces of lines measured 2-3x slower there).  The 16
// possible decoded values of each row — (K3[n&7] + re*(+-1)) * ks for
// turbo_prod K, V4[n] * rms otherwise, with the reference's exact operations
// — are tabulated per row in LDS and looked up per nibble.  Waves are
// persistent: each walks groups of 64/LPR rows with the next group's slot and
// codes in flight while it transforms and stores the current one.
// ---------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The layers one dequant launch covers (pools and outputs of each; one slot
// mapping shared by all), passed by value in the kernel arguments.
template <int ML>
struct LayerSet {
    const uint8_t* pool[ML];
    uint16_t* out_key[ML];
    uint16_t* out_value[ML];
};
constexpr int kMaxLayersPerLaunch = 64;
// Launch shapes (workgroups per CU; measured on 32K-token, two-head layers).
// The four-lanes-per-row kernel, one layer per launch (D = 32, 64, QJL,
// buffers not 16-byte aligned): up to four persistent workgroups per CU.
#ifndef TQ_DEQ_BLOCKS_PER_CU
#define TQ_DEQ_BLOCKS_PER_CU 4
#endif
// The four-lanes-per-row kernel, several layers per launch (D = 128 with
// unaligned buffers): 32 KB of LDS per workgroup lets 4 reside per CU; a
// grid of several such rounds balances the tail (36 layers: 4 per CU
// 9.3 us/layer, 8: 9.0, 24: 8.6, 48-192: 8.8-9.0).
#ifndef TQ_DEQ_LAYERS_BLOCKS_PER_CU
#define TQ_DEQ_LAYERS_BLOCKS_PER_CU 24
#endif
// A row per lane, several layers per launch: two workgroups reside per CU; a
// grid of several rounds balances the tail (36 layers: 2 per CU 8.5 us/layer,
// 8: 8.2, 16-64: 7.9-8.0).
#ifndef TQ_DEQ_ROWS_BLOCKS_PER_CU
#define TQ_DEQ_ROWS_BLOCKS_PER_CU 24
#endif
// Half a row per lane, one layer per launch (a layer needs 512: two per CU,
// all resident).
#ifndef TQ_DEQ_ONE_BLOCKS_PER_CU
#define TQ_DEQ_ONE_BLOCKS_PER_CU 8
#endif

// SCH: 0 turbo_mse, 1 turbo_prod, 2 the reference's unexported QJL-1b page
// (tq_qjl_kernels.cu:189-245): K = +-ks per sign bit, fed through the same
// per-row table as 0/1 "nibbles" (the sign byte's bits spread one per
// nibble), and the rotation's sign flip (-1)^i has no head term.
// ML > 1: num_layers <= ML layers in one launch; the persistent waves walk
// (layer, row group) pairs, layer-major, so the launch and the first-code
// latency are paid once for all of them.
template <int D, int SCH, int ML = 1>
__global__ __launch_bounds__(kBlock) void dequant_stream_kernel(
    const LayerSet<ML> layers, const int32_t* __restrict__ slots, PageGeom g, int num_rows,
    int num_layers, float inv, OutLayout ol) {
    constexpr bool PROD = SCH == 1, QJL = SCH == 2;
    static_assert(!QJL || D == 128, "QJL: D = 128");
    constexpr int E = 32;           // elements per lane
    constexpr int LPR = D / E;      // lanes per row
    constexpr int RPW = 64 / LPR;   // rows per wave group
    // Each lane keeps a private copy of its row's two 16-entry tables: entry n
    // of (wave w, lane l) is word ((n*4 + w)*64 + l), so every lookup of lane l
    // hits LDS bank l and a wave's 64 lookups never conflict, whatever the
    // nibbles.  The entry's byte address is 4l + 256*(4n + w): the lane's base
    // with byte 1 replaced by 4n + w (one v_perm_b32).  V follows K by 16 KiB.
    constexpr int kWaves = kBlock / 64;
    static_assert(kWaves == 4, "byte 1 of a table address holds 4*nibble + wave");
    constexpr uint32_t kTabBytes = 16 * kWaves * 64 * sizeof(float);
    // The kernel's only LDS object, so it starts at LDS address 0 and the
    // address bits above byte 1 are those of the 16 KiB table offset alone.
    __shared__ __attribute__((aligned(1024))) float tab[2][16][kWaves][64];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane % LPR, rw = lane / LPR;
    float* TK = &tab[0][0][wave][lane];  // entry n at TK[n * kWaves * 64]
    float* TV = &tab[1][0][wave][lane];
    const uint32_t tbase = (uint32_t)reinterpret_cast<uintptr_t>((lds_float*)TK);
    const uint32_t wsplat = 0x01010101u * (uint32_t)wave;
    const int groups = (num_rows + RPW - 1) / RPW;  // row groups per layer
    const int total = groups * num_layers;          // (layer, group) pairs
    const int stride = gridDim.x * (kBlock / 64);

    struct Item {
        uint4 kw, vw;
        float ks, re, vs;
        int row, t, h;
        int pt, ph;  // token and head of row ^ 1 (the store partner when LPR = 4)
        int layer;   // wave-uniform
        bool live, plive;
    };
    // pair index -> (layer, group of the layer); wave-uniform
    auto split_pair = [&](int gi, int& grp) -> int {
        if constexpr (ML == 1) {
            grp = gi;
            return 0;
        } else {
            const int l = gi / groups;
            grp = gi - l * groups;
            return l;
        }
    };
    auto token_head = [&](int row, int& t, int& h) {
        if (g.h_shift >= 0) {
            t = row >> g.h_shift;
            h = row & (g.H - 1);
        } else {
            t = row / g.H;
            h = row - t * g.H;
        }
    };
    auto load_slot = [&](int gi) -> int {
        if (gi >= total) return -1;
        int grp;
        split_pair(gi, grp);
        const int row = grp * RPW + rw;
        if (row >= num_rows) return -1;
        int t, h;
        token_head(row, t, h);
        return slots[t];
    };
    auto fetch = [&](int gi, int slot) -> Item {
        Item it;
        int grp;
        it.layer = __builtin_amdgcn_readfirstlane(gi < total ? split_pair(gi, grp) : 0);
        if (gi >= total) grp = groups;
        const uint8_t* pool = layers.pool[it.layer];
        it.row = grp * RPW + rw;
        token_head(min(it.row, num_rows - 1), it.t, it.h);
        it.live = gi < total && it.row < num_rows && slot >= 0;
        it.kw = make_uint4(0, 0, 0, 0);
        it.vw = it.kw;
        it.ks = it.re = it.vs = 0.0f;
        if (it.live) {
            int page, tib;
            split_slot(slot, g, page, tib);
            const size_t cell = (size_t)(tib * g.H + it.h);
            const uint8_t* base = pool + (size_t)page * g.page_size;
            // dword j + LPR*m of the cell holds the nibbles of chunk m
            const uint32_t* kp =
                reinterpret_cast<const uint32_t*>(base + g.kc_off + cell * g.code_stride) + j;
            const uint32_t* vp =
                reinterpret_cast<const uint32_t*>(base + g.vc_off + cell * g.code_stride) + j;
            if constexpr (QJL) {
                // sign byte j + 4m (elements 8(j + 4m) .. + 7) spread to one
                // bit per nibble: nibble i = bit i
                const uint8_t* kb = base + g.kc_off + cell * (D / 8) + j;
                const auto spread = [](uint32_t b) {
                    b = (b | (b << 12)) & 0x000F000Fu;
                    b = (b | (b << 6)) & 0x03030303u;
                    return (b | (b << 3)) & 0x11111111u;
                };
                it.kw = make_uint4(spread(kb[0]), spread(kb[4]), spread(kb[8]), spread(kb[12]));
            } else {
                it.kw = make_uint4(kp[0], kp[LPR], kp[2 * LPR], kp[3 * LPR]);
            }
            it.vw = make_uint4(vp[0], vp[LPR], vp[2 * LPR], vp[3 * LPR]);
            it.ks = h2f(ld_u16(base + g.ks_off + cell * g.scale_stride));
            it.vs = h2f(ld_u16(base + g.vs_off + cell * g.scale_stride));
            if (PROD) it.re = h2f(ld_u16(base + g.kres_off + cell * g.scale_stride));
        }
        if constexpr (LPR == 4) {
            token_head(min(it.row ^ 1, num_rows - 1), it.pt, it.ph);
            it.plive = lane_xor<4>(it.live ? 1.0f : 0.0f) != 0.0f;
        }
        return it;
    };

    // One tensor at a time keeps 32 values live per lane.
    auto transform = [&](const Item& it, uint4 w, uint32_t toff, uint16_t* out) {
        float x[E];
        const uint32_t wa[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            // bytes 4*nibble + wave, for even and odd elements
            const uint32_t ev = ((wa[q] << 2) & 0x3C3C3C3Cu) | wsplat;
            const uint32_t od = ((wa[q] >> 2) & 0x3C3C3C3Cu) | wsplat;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                // byte 0 and bytes 2..3 from tbase, byte 1 = 4*nibble + wave.
                const uint32_t sel = 0x03020000u | ((uint32_t)(4 + b) << 8);
                const uint32_t ae = __builtin_amdgcn_perm(ev, tbase, sel) + toff;
                const uint32_t ao = __builtin_amdgcn_perm(od, tbase, sel) + toff;
                x[8 * q + 2 * b] = *reinterpret_cast<const lds_float*>(ae);
                x[8 * q + 2 * b + 1] = *reinterpret_cast<const lds_float*>(ao);
            }
        }
        // x[8m + i] is element 8*(j + LPR*m) + i.  Stages in the reference's
        // order: len = 1, 2, 4 pair k and k ^ len in the lane ...
        auto reg_stage = [&](int kb) {
#pragma unroll
            for (int k = 0; k < E; ++k) {
                if ((k & kb) == 0) {
                    const float a = x[k], b = x[k + kb];
                    x[k] = a + b;
                    x[k + kb] = a - b;
                }
            }
        };
        reg_stage(1);
        reg_stage(2);
        reg_stage(4);
        // ... len = 8, 16 (LPR = 4; 8 for LPR = 2) pair lanes j and j ^ 1,
        // j ^ 2.  The lower lane needs mine + partner, the upper partner -
        // mine: fmaf(mine, +-1, partner) is both, exactly (exact product, one
        // rounding of the sum) ...
        if constexpr (LPR >= 2) {
            const float sg = (j & 1) ? -1.0f : 1.0f;
#pragma unroll
            for (int k = 0; k < E; ++k) x[k] = fmaf(x[k], sg, quad_xor<1>(x[k]));
        }
        if constexpr (LPR >= 4) {
            const float sg = (j & 2) ? -1.0f : 1.0f;
#pragma unroll
            for (int k = 0; k < E; ++k) x[k] = fmaf(x[k], sg, quad_xor<2>(x[k]));
        }
        // ... and the two largest (chunk m ^ 1, m ^ 2) are in the lane again.
        reg_stage(8);
        reg_stage(16);
        // Element 8*(j + LPR*m) + i has sign (-1)^(i + h) ((-1)^i for QJL).
        const float se = (!QJL && (it.h & 1)) ? -inv : inv;
        u32x4 v[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const float* c = x + 8 * m;
            v[m] = u32x4{f2h2(c[0] * se, c[1] * -se), f2h2(c[2] * se, c[3] * -se),
                         f2h2(c[4] * se, c[5] * -se), f2h2(c[6] * se, c[7] * -se)};
        }
        if constexpr (LPR == 4) {
            // Streaming (non-temporal) stores of whole 128-byte lines: the
            // fp16 output is written once and is far larger than the caches,
            // and a line that reaches the L2 in two non-temporal pieces is
            // written to memory twice.  Rows 2p and 2p + 1 (lanes 8p..8p+3
            // and 8p+4..8p+7) trade half their chunks across lane ^ 4, so
            // store k writes line k >> 1 of row 2p + (k & 1) with all 8
            // lanes: lane j of the even row chunk j, of the odd row chunk
            // 4 + j (of the line).
            const int odd = rw & 1;
            const u32x4 s0 = odd ? v[0] : v[1], s1 = odd ? v[2] : v[3];
            u32x4 r0, r1;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                r0[q] = __float_as_uint(lane_xor<4>(__uint_as_float(s0[q])));
                r1[q] = __float_as_uint(lane_xor<4>(__uint_as_float(s1[q])));
            }
            // store k: own row when (k & 1) == odd, else the partner's
            const u32x4 val[4] = {odd ? r0 : v[0], odd ? v[1] : r0, odd ? r1 : v[2],
                                  odd ? v[3] : r1};
            uint4* const mine = reinterpret_cast<uint4*>(out + ol.offset(it.t, it.h));
            uint4* const other = reinterpret_cast<uint4*>(out + ol.offset(it.pt, it.ph));
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const bool own = (k & 1) == odd;
                if (own ? it.live : it.plive)
                    __builtin_nontemporal_store(
                        val[k], reinterpret_cast<u32x4*>((own ? mine : other) + 8 * (k >> 1) +
                                                         4 * odd + j));
            }
        } else {
            if (!it.live) return;
            uint4* d = reinterpret_cast<uint4*>(out + ol.offset(it.t, it.h)) + j;
#pragma unroll
            for (int m = 0; m < 4; ++m) reinterpret_cast<u32x4*>(d + LPR * m)[0] = v[m];
        }
    };

    int gi = blockIdx.x * (kBlock / 64) + wave;
    Item cur = fetch(gi, load_slot(gi));
    int s_next = load_slot(gi + stride);
    while (gi < total) {  // wave-uniform
        const Item nxt = fetch(gi + stride, s_next);
        s_next = load_slot(gi + 2 * stride);
        // Every lane writes all 16 entries of its own copies (one b32 store
        // per entry and tensor; a wave's 64 stores fill 64 distinct banks).
        {
            float* myK = &tab[0][0][wave][lane];
            float* myV = &tab[1][0][wave][lane];
#pragma unroll
            for (int n = 0; n < 16; ++n) {
                const float kv =
                    QJL ? ((n & 1) ? cur.ks : -cur.ks)
                    : PROD ? (kK3[n & 7] + cur.re * ((n & 8) ? 1.0f : -1.0f)) * cur.ks
                           : kV4[n] * cur.ks;
                myK[n * kWaves * 64] = kv;
                myV[n * kWaves * 64] = kV4[n] * cur.vs;
            }
        }
        // The table is private to this wave: wave-scope ordering suffices.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        transform(cur, cur.kw, 0, layers.out_key[cur.layer]);
        transform(cur, cur.vw, kTabBytes, layers.out_value[cur.layer]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        cur = nxt;
        gi += stride;
    }
}

// ---------------------------------------------------------------------------
// Dequant, one row (E = 128) or half a row (E = 64) per lane (D = 128;
// turbo_prod and turbo_mse).  With a whole row every WHT stage and both
// decode tables stay inside the lane: no cross-lane butterfly (a DPP move
// plus an fmac per value per stage) and one table build per row instead of
// one per lane of a row: 45 VALU instructions per row against 72 for the
// four-lanes-per-row form, which is VALU-bound here.  Half a row per lane
// (52 per row) keeps one DPP stage and twice the waves, for launches with
// few row groups.  Lane l of a wave group owns row 64*group + l (E = 64:
// half l % 2 of row 32*group + l / 2); it loads its E/2 code bytes per
// tensor as 16-byte loads.  The outputs leave one 128-byte line per lane at
// a time: each lane writes its line into a padded wave-private LDS stage
// (144-byte rows: the 16-byte writes of eight consecutive lanes cover the
// 32 banks once) with the line's byte offset in the layer's output, then
// store r of the wave writes the lines of lanes 8r .. 8r + 7, eight whole
// lines per buffer store.  Waves walk (layer, row group) pairs grid-stride
// with the next pair's slot, codes and scales in flight.
// ---------------------------------------------------------------------------
constexpr int kRowStageBytes = 144;  // staged bytes per lane: one output line + 16 of pad
// The row kernels store through buffer descriptors of a layer's output,
// num_rows * 256 bytes each: a skipped row's byte offset is kBufSkip, past
// the end of every buffer the launchers allow (rows up to kBufMaxRows), so
// the hardware's range check drops its stores without a branch.
constexpr uint32_t kBufSkip = 0x80000000u;
constexpr int kBufMaxRows = (int)(kBufSkip / 256u) - 1;
constexpr uint32_t kBufWord3 = 0x00020000u;  // descriptor word 3 on gfx9: 32-bit data format
// Row-per-lane dequant: staged output lines (and their row offsets) read
// from LDS this many stores ahead of the store that writes them, 1..7 (36
// layers of 32K tokens in one launch: 8.20 us per layer with each read just
// before its store, 7.86 with 2; 1, 3 and 7 within 0.1 us of 2).
#ifndef TQ_DEQ_STORE_AHEAD
#define TQ_DEQ_STORE_AHEAD 2
#endif
constexpr int kStoreAhead = TQ_DEQ_STORE_AHEAD;
static_assert(kStoreAhead >= 1 && kStoreAhead <= 7, "1 to 7 stores ahead");

template <int SCH, int ML, int E>
__global__ __launch_bounds__(kBlock, 2) void dequant_rows_kernel(
    const LayerSet<ML> layers, const int32_t* __restrict__ slots, PageGeom g, int num_rows,
    int num_layers, float inv, OutLayout ol) {
    constexpr bool PROD = SCH == 1;
    static_assert(SCH == 0 || SCH == 1, "turbo_mse or turbo_prod pages");
    // E = 128: lane l owns row l of the group's 64; E = 64: lanes 2r and
    // 2r + 1 own halves 0 and 1 (elements 64j .. 64j + 63) of row r of 32, and
    // the last WHT stage (len = 64) pairs them across the lane pair.
    static_assert(E == 128 || E == 64, "a whole row or half a row per lane");
    constexpr int LPR = 128 / E;   // lanes per row
    constexpr int RPG = 64 / LPR;  // rows per wave group
    constexpr int NQ = E / 32;     // 16-byte code loads per tensor and lane
    constexpr int kWaves = kBlock / 64;
    static_assert(kWaves == 4, "byte 1 of a table address holds 4*nibble + wave");
    // Tables as in dequant_stream_kernel: entry n of (wave w, lane l) is word
    // (n*4 + w)*64 + l of the tensor's 16 KiB, K first; then one stage per
    // wave, one kRowStageBytes row per lane: the lane's output line (bytes
    // 0..127) and the byte offset of its K and V output rows in their
    // buffers (bytes 128..131; kBufSkip for a row not written).  68 KB per
    // workgroup.  (One table shared by K and V, the V table written after
    // the K transform, takes 52 KB: per-layer launches alone ran 1% faster,
    // but with three such workgroups per CU the decode attention's 82.5 KB
    // workgroups found no room beside them: the two-stream step went from
    // 0.55 to 0.60 ms.)
    constexpr uint32_t kTabBytes = 16 * kWaves * 64 * sizeof(float);
    constexpr uint32_t kStageBytes = 64 * kRowStageBytes;
    // The kernel's only LDS object: it starts at LDS address 0, so byte 1 of
    // an entry's address is 4*nibble + wave and the bytes above it are zero.
    __shared__ __attribute__((aligned(1024))) uint32_t lds[(2 * kTabBytes + kWaves * kStageBytes) / 4];
    typedef __attribute__((address_space(3))) u32x4 lds_u32x4;

    const int lane = threadIdx.x & 63;
    const int half_j = LPR == 2 ? (lane & 1) : 0;  // the half of the row this lane owns
    const int rw = LPR == 2 ? (lane >> 1) : lane;   // its row in the group
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((lds_float*)(void*)lds);
    const uint32_t tbase = lds0 + 4u * lane + 256u * wave;  // entry 0 of this lane's K table
    const uint32_t wsplat = 0x01010101u * (uint32_t)wave;
    const uint32_t stage = lds0 + 2 * kTabBytes + wave * kStageBytes;
    const uint32_t my_row = stage + lane * kRowStageBytes;        // staged by this lane
    const uint32_t rd_row = stage + (lane >> 3) * kRowStageBytes;  // read by store 0 (+ 8 rows per store)
    const int groups = (num_rows + RPG - 1) / RPG;  // row groups per layer
    const int total = groups * num_layers;    // (layer, group) pairs
    const int stride = gridDim.x * kWaves;

    // A group's cell: this lane's row, its page and cell, and whether it is
    // written.  Loads are branch-free (so the in-order vector-memory counter
    // never waits on a later load early): a row not written reads the first
    // bytes of its layer's K output instead (valid memory; the values are
    // not used).
    struct Loc {
        const uint8_t* base;   // page start
        const uint8_t* dummy;  // the layer's first output row
        int cell;              // tib * H + h
        int row, layer;        // layer wave-uniform
        bool live;
    };
    auto split_pair = [&](int gi, int& grp) -> int {
        if constexpr (ML == 1) {
            grp = gi;
            return 0;
        } else {
            const int l = gi / groups;
            grp = gi - l * groups;
            return l;
        }
    };
    auto token_head = [&](int row, int& t, int& h) {
        if (g.h_shift >= 0) {
            t = row >> g.h_shift;
            h = row & (g.H - 1);
        } else {
            t = row / g.H;
            h = row - t * g.H;
        }
    };
    // (branch-free and unchecked: past the end it reads the slot of the last
    // row, which locate does not use)
    auto load_slot = [&](int gi) -> int {
        int grp;
        split_pair(min(gi, total - 1), grp);
        int t, h;
        token_head(min(grp * RPG + rw, num_rows - 1), t, h);
        return slots[t];
    };
    auto locate = [&](int gi, int slot) -> Loc {
        Loc c;
        int grp = groups;
        c.layer = gi < total ? split_pair(gi, grp) : 0;
        c.row = grp * RPG + rw;
        c.live = gi < total && c.row < num_rows && slot >= 0;
        int t, h, page, tib;
        token_head(min(c.row, num_rows - 1), t, h);
        split_slot(c.live ? slot : 0, g, page, tib);
        c.cell = tib * g.H + h;
        c.base = layers.pool[c.layer] + (size_t)page * g.page_size;
        c.dummy = reinterpret_cast<const uint8_t*>(layers.out_key[c.layer]);
        return c;
    };
    // The lane's E/2 code bytes of the row (dword 4q + e of them holds
    // elements 64j + 8(4q + e) .. + 7).
    auto load_codes = [&](const Loc& c, uint64_t off, uint4 (&w)[NQ]) {
        const uint4* p = reinterpret_cast<const uint4*>(
            c.live ? c.base + off + (size_t)c.cell * 64 + 32 * half_j : c.dummy);
#pragma unroll
        for (int q = 0; q < NQ; ++q) w[q] = p[q];
    };
    struct Scales {
        uint32_t ks, re, vs;  // raw fp16 in the low halves (converted when used)
    };
    auto load_scales = [&](const Loc& c, Scales& sc) {
        const uint8_t* p = c.base + (size_t)c.cell * g.scale_stride;
        sc.ks = ld_u16(c.live ? p + g.ks_off : c.dummy);
        sc.vs = ld_u16(c.live ? p + g.vs_off : c.dummy);
        sc.re = PROD ? ld_u16(c.live ? p + g.kres_off : c.dummy) : 0u;
    };

    // Decode, transform and store one tensor of the group (toff: its table;
    // rs: the tensor's output in this layer as a buffer).
    auto transform = [&](const uint4 (&cw)[NQ], uint32_t toff, float se,
                         __amdgpu_buffer_rsrc_t rs) {
        float x[E];
#pragma unroll
        for (int c = 0; c < E / 8; ++c) {
            const uint4 q = cw[c / 4];
            const uint32_t w = c % 4 == 0 ? q.x : c % 4 == 1 ? q.y : c % 4 == 2 ? q.z : q.w;
            // bytes 4*nibble + wave, for even and odd elements
            const uint32_t ev = ((w << 2) & 0x3C3C3C3Cu) | wsplat;
            const uint32_t od = ((w >> 2) & 0x3C3C3C3Cu) | wsplat;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                // bytes 0, 2, 3 from tbase, byte 1 = 4*nibble + wave
                const uint32_t sel = 0x03020000u | ((uint32_t)(4 + b) << 8);
                const uint32_t ae = __builtin_amdgcn_perm(ev, tbase, sel) + toff;
                const uint32_t ao = __builtin_amdgcn_perm(od, tbase, sel) + toff;
                x[8 * c + 2 * b] = *reinterpret_cast<const lds_float*>(ae);
                x[8 * c + 2 * b + 1] = *reinterpret_cast<const lds_float*>(ao);
            }
            // (each dword's addresses die at its lookups: 128 live addresses
            // on top of the 128 values would not fit two waves per SIMD)
            __builtin_amdgcn_sched_barrier(0);
        }
        // The reference's stages in its order, len = 1, 2, ..., 64: in the
        // lane up to E / 2 ...
#pragma unroll
        for (int len = 1; len < E; len *= 2) {
#pragma unroll
            for (int k = 0; k < E; ++k) {
                if ((k & len) == 0) {
                    const float a = x[k], b = x[k + len];
                    x[k] = a + b;
                    x[k + len] = a - b;
                }
            }
        }
        // ... and len = 64 across the lane pair: the lower half needs mine +
        // partner, the upper partner - mine, both fmaf(mine, +-1, partner)
        // exactly (exact product, one rounding of the sum).
        if constexpr (LPR == 2) {
            const float sg = half_j ? -1.0f : 1.0f;
#pragma unroll
            for (int k = 0; k < E; ++k) x[k] = fmaf(x[k], sg, quad_xor<1>(x[k]));
        }
        // Element e has sign (-1)^(e + h): se for even e, -se for odd (64j is
        // even).  Each lane's E outputs are E / 64 lines of 128 bytes.
#pragma unroll
        for (int half = 0; half < E / 64; ++half) {
            const float* c = x + 64 * half;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                *reinterpret_cast<lds_u32x4*>(my_row + 16 * k) =
                    u32x4{f2h2(c[8 * k] * se, c[8 * k + 1] * -se),
                          f2h2(c[8 * k + 2] * se, c[8 * k + 3] * -se),
                          f2h2(c[8 * k + 4] * se, c[8 * k + 5] * -se),
                          f2h2(c[8 * k + 6] * se, c[8 * k + 7] * -se)};
            // The stage is private to this wave: wave-scope ordering suffices.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // Store r's line and row offset are read kStoreAhead stores
            // ahead, so the LDS round trips overlap the stores instead of
            // preceding each one.
            constexpr int P = kStoreAhead;
            u32x4 vr[P + 1];
            uint32_t ar[P + 1];
            auto read = [&](int r) {
                const uint32_t src = rd_row + 8 * r * kRowStageBytes;
                vr[r % (P + 1)] = *reinterpret_cast<const lds_u32x4*>(src + 16 * (lane & 7));
                ar[r % (P + 1)] = *reinterpret_cast<const lds_u32*>(src + 128);
            };
#pragma unroll
            for (int r = 0; r < P; ++r) read(r);
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                if (r + P < 8) read(r + P);
                // (aux 2: non-temporal)
                __builtin_amdgcn_raw_buffer_store_b128(
                    vr[r % (P + 1)], rs, ar[r % (P + 1)] + 128 * half + 16 * (lane & 7), 0, 2);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    };

    // Loads in flight for half a group each: this group's V codes during its
    // K transform; the next group's K codes, scales and the slot after it
    // during its V transform.  Each lands in the registers its previous
    // contents left (no copies, which would wait for the loads).
    int gi = blockIdx.x * kWaves + wave;
    Loc cur = locate(gi, load_slot(gi));
    uint4 kw[NQ], vw[NQ];
    Scales sc;
    load_codes(cur, g.kc_off, kw);
    load_scales(cur, sc);
    int s_next = load_slot(gi + stride);
    while (gi < total) {  // wave-uniform
        load_codes(cur, g.vc_off, vw);
        const Loc nxt = locate(gi + stride, s_next);
        // This lane's row: its tables (16 entries per tensor, the reference's
        // exact operations) and its output offset for the stores.
        {
            const float ks = h2f(sc.ks), vs = h2f(sc.vs), re = h2f(sc.re);
#pragma unroll
            for (int n = 0; n < 16; ++n) {
                const float kv = PROD ? (kK3[n & 7] + re * ((n & 8) ? 1.0f : -1.0f)) * ks
                                      : kV4[n] * ks;
                *reinterpret_cast<lds_float*>(tbase + 1024u * n) = kv;
                *reinterpret_cast<lds_float*>(tbase + kTabBytes + 1024u * n) = kV4[n] * vs;
            }
        }
        int t, h;
        token_head(min(cur.row, num_rows - 1), t, h);
        const uint64_t eo = ol.offset(t, h) + 64 * half_j;  // element offset of the lane's line
        *reinterpret_cast<lds_u32*>(my_row + 128) = cur.live ? (uint32_t)(2 * eo) : kBufSkip;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const float se = (h & 1) ? -inv : inv;  // s(2j, h) * inv; s(2j+1, h) = -s(2j, h)
        // The layer's K and V outputs as buffers of num_rows * 256 bytes
        // (below kBufSkip: the launchers' row limit).
        const int lyr = __builtin_amdgcn_readfirstlane(cur.layer);
        const uint32_t out_bytes = (uint32_t)num_rows * 256u;
        transform(kw, 0, se,
                  __builtin_amdgcn_make_buffer_rsrc(layers.out_key[lyr], 0, out_bytes, kBufWord3));
        load_codes(nxt, g.kc_off, kw);
        load_scales(nxt, sc);
        s_next = load_slot(gi + 2 * stride);
        transform(vw, kTabBytes, se,
                  __builtin_amdgcn_make_buffer_rsrc(layers.out_value[lyr], 0, out_bytes, kBufWord3));
        cur = nxt;
        gi += stride;
    }
}

// The row-per-lane kernel reads codes as 16-byte pieces.
bool rows_dequant_ok(const PageGeom& g, const void* pool, const void* ok, const void* ov) {
    const auto al = [](uint64_t v, uint64_t a) { return (v & (a - 1)) == 0; };
    return g.D == 128 && g.code_stride == 64 && al(g.page_size, 16) && al(g.kc_off, 16) &&
           al(g.vc_off, 16) && al(g.ks_off, 2) && al(g.vs_off, 2) && al(g.kres_off, 2) &&
           al(reinterpret_cast<uintptr_t>(pool), 16) &&
           al(reinterpret_cast<uintptr_t>(ok), 16) && al(reinterpret_cast<uintptr_t>(ov), 16);
}

// The streaming kernel reads codes as dwords and writes 16-byte output chunks.
bool wide_dequant_ok(const PageGeom& g, const void* pool, const void* ok, const void* ov) {
    const auto al = [](uint64_t v, uint64_t a) { return (v & (a - 1)) == 0; };
    return (g.D == 32 || g.D == 64 || g.D == 128) && al(g.page_size, 4) && al(g.kc_off, 4) &&
           al(g.vc_off, 4) && al(reinterpret_cast<uintptr_t>(pool), 4) &&
           al(reinterpret_cast<uintptr_t>(ok), 16) && al(reinterpret_cast<uintptr_t>(ov), 16);
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
    const auto al = [](uint64_t v, uint64_t a) { return (v & (a - 1)) == 0; };
    if ((g.D == 64 || g.D == 128) && al(g.kc_off, 4) && al(g.vc_off, 4) && al(g.page_size, 4) &&
        al(reinterpret_cast<uintptr_t>(pool), 4) && al(reinterpret_cast<uintptr_t>(key), 4) &&
        al(reinterpret_cast<uintptr_t>(value), 4)) {
        constexpr int R = kPackLanes;
        const dim3 wgrid((rows + kBlock / R - 1) / (kBlock / R));
        const bool prod = s == Scheme::Prod;
        const PackSet<1> one{{key}, {value}, {pool}};
        auto go = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, wgrid, dim3(kBlock), 0, stream, one, slots, g, rows, inv);
        };
        if (g.D == 128) prod ? go(pack_wide_kernel<128, 1>) : go(pack_wide_kernel<128, 0>);
        else prod ? go(pack_wide_kernel<64, 1>) : go(pack_wide_kernel<64, 0>);
        check_launch(prod ? "turbo_prod_pack_kv_kernel" : "turbo_mse_pack_kv_kernel");
        return;
    }
    if (s == Scheme::Prod) {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(prod_pack_kernel<kD>, grid, dim3(kBlock), 0, stream,
                                              key, value, slots, pool, g, rows, inv, PackDebug{}));
        check_launch("turbo_prod_pack_kv_kernel");
    } else {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(mse_pack_kernel<kD>, grid, dim3(kBlock), 0, stream,
                                              key, value, slots, pool, g, rows, inv));
        check_launch("turbo_mse_pack_kv_kernel");
    }
}

void launch_prod_pack_debug(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                            uint8_t* pool, const PageGeom& g, int num_tokens, const PackDebug& dbg,
                            hipStream_t stream) {
    const int rows = num_tokens * g.H;
    if (rows <= 0) return;
    // (debug buffers are written as float2 / int2 pairs)
    const auto al8 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; };
    if (!al8(dbg.k_rot) || !al8(dbg.v_rot) || !al8(dbg.kn) || !al8(dbg.vn) || !al8(dbg.kidx) ||
        !al8(dbg.vidx))
        throw Error("turbo_prod pack debug: debug buffers must be 8-byte aligned");
    const int rpb = kBlock / (g.D / 2);
    const dim3 grid((rows + rpb - 1) / rpb);
    const float inv = inv_sqrt_d(g.D);
    TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(prod_pack_kernel<kD>, grid, dim3(kBlock), 0, stream, key,
                                          value, slots, pool, g, rows, inv, dbg));
    check_launch("turbo_prod_pack_kv_kernel");
}

void launch_pack_layers(Scheme s, const uint16_t* const* keys, const uint16_t* const* values,
                        const int32_t* slots, uint8_t* const* pools, const PageGeom& g,
                        int num_tokens, int num_layers, hipStream_t stream) {
    const int rows = num_tokens * g.H;
    if (rows <= 0 || num_layers <= 0) return;
    const auto al = [](uint64_t v, uint64_t a) { return (v & (a - 1)) == 0; };
    bool wide = (g.D == 64 || g.D == 128) && al(g.kc_off, 4) && al(g.vc_off, 4) &&
                al(g.page_size, 4);
    for (int l = 0; l < num_layers && wide; ++l)
        wide = al(reinterpret_cast<uintptr_t>(pools[l]), 4) &&
               al(reinterpret_cast<uintptr_t>(keys[l]), 4) &&
               al(reinterpret_cast<uintptr_t>(values[l]), 4);
    if (!wide) {  // the per-layer kernels (other head dims, unaligned buffers)
        for (int l = 0; l < num_layers; ++l)
            launch_pack(s, keys[l], values[l], slots, pools[l], g, num_tokens, stream);
        return;
    }
    const float inv = inv_sqrt_d(g.D);
    const bool prod = s == Scheme::Prod;
    constexpr int R = kPackLanes, ML = kMaxPackLayersPerLaunch;
    for (int l0 = 0; l0 < num_layers; l0 += ML) {
        const int n = std::min(ML, num_layers - l0);
        PackSet<ML> set{};
        for (int l = 0; l < n; ++l) {
            set.key[l] = keys[l0 + l];
            set.value[l] = values[l0 + l];
            set.pool[l] = pools[l0 + l];
        }
        const dim3 grid((rows + kBlock / R - 1) / (kBlock / R), n);
        auto go = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, grid, dim3(kBlock), 0, stream, set, slots, g, rows, inv);
        };
        if (g.D == 128)
            prod ? go(pack_wide_kernel<128, 1, ML>) : go(pack_wide_kernel<128, 0, ML>);
        else
            prod ? go(pack_wide_kernel<64, 1, ML>) : go(pack_wide_kernel<64, 0, ML>);
        check_launch(prod ? "turbo_prod_pack_kv_layers" : "turbo_mse_pack_kv_layers");
    }
}

bool launch_qjl_wide_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                          uint8_t* pool, const QjlGeom& q, int num_tokens, hipStream_t stream) {
    const auto al = [](uint64_t v, uint64_t a) { return (v & (a - 1)) == 0; };
    if (!((q.D == 64 || q.D == 128) && q.k1_bytes == q.D / 8 && q.v4_bytes == q.D / 2 &&
          al(q.ks_off, 2) && al(q.vs_off, 2) && al(q.page_size, 2) &&
          al(reinterpret_cast<uintptr_t>(key), 4) && al(reinterpret_cast<uintptr_t>(value), 4)))
        return false;
    const int rows = num_tokens * q.H;
    if (rows <= 0) return true;
    PageGeom g{};
    g.page_size = q.page_size;
    g.kc_off = q.k1_off;
    g.vc_off = q.v4_off;
    g.ks_off = q.ks_off;
    g.vs_off = q.vs_off;
    g.code_stride = q.v4_bytes;  // V rows; the K sign rows are D/8 bytes
    g.scale_stride = 2;
    g.H = q.H;
    g.D = q.D;
    g.block_size = q.block_size;
    g.bs_shift = (q.block_size & (q.block_size - 1)) == 0 ? __builtin_ctz(q.block_size) : -1;
    g.h_shift = (q.H & (q.H - 1)) == 0 ? __builtin_ctz(q.H) : -1;
    const dim3 grid((rows + kBlock / kPackLanes - 1) / (kBlock / kPackLanes));
    const float inv = inv_sqrt_d(g.D);
    const PackSet<1> one{{key}, {value}, {pool}};
    if (g.D == 128)
        hipLaunchKernelGGL((pack_wide_kernel<128, 2>), grid, dim3(kBlock), 0, stream, one, slots, g,
                           rows, inv);
    else
        hipLaunchKernelGGL((pack_wide_kernel<64, 2>), grid, dim3(kBlock), 0, stream, one, slots, g,
                           rows, inv);
    check_launch("qjl_pack_kv_kernel");
    return true;
}

bool launch_qjl_stream_dequant(const uint8_t* pool, const int32_t* slots, uint16_t* out_key,
                               uint16_t* out_value, const QjlGeom& q, int num_tokens,
                               hipStream_t stream) {
    const auto al = [](uint64_t v, uint64_t a) { return (v & (a - 1)) == 0; };
    if (!(q.D == 128 && q.k1_bytes == 16 && q.v4_bytes == 64 && al(q.page_size, 4) &&
          al(q.v4_off, 4) && al(q.ks_off, 2) && al(q.vs_off, 2) &&
          al(reinterpret_cast<uintptr_t>(pool), 4) && al(reinterpret_cast<uintptr_t>(out_key), 16) &&
          al(reinterpret_cast<uintptr_t>(out_value), 16)))
        return false;
    const int rows = num_tokens * q.H;
    if (rows <= 0) return true;
    PageGeom g{};
    g.page_size = q.page_size;
    g.kc_off = q.k1_off;
    g.vc_off = q.v4_off;
    g.ks_off = q.ks_off;
    g.vs_off = q.vs_off;
    g.code_stride = q.v4_bytes;  // V rows; the K sign rows are D/8 = 16 bytes
    g.scale_stride = 2;
    g.H = q.H;
    g.D = q.D;
    g.block_size = q.block_size;
    g.bs_shift = (q.block_size & (q.block_size - 1)) == 0 ? __builtin_ctz(q.block_size) : -1;
    g.h_shift = (q.H & (q.H - 1)) == 0 ? __builtin_ctz(q.H) : -1;
    OutLayout ol;
    ol.tok = (uint64_t)g.H * g.D;
    ol.head = (uint64_t)g.D;
    const int rows_per_block = kBlock / (g.D / 32);
    const int blocks_needed = (rows + rows_per_block - 1) / rows_per_block;
    const dim3 grid(std::max(1, std::min(blocks_needed, 4 * num_cus())));
    const LayerSet<1> one{{pool}, {out_key}, {out_value}};
    hipLaunchKernelGGL((dequant_stream_kernel<128, 2>), grid, dim3(kBlock), 0, stream, one, slots,
                       g, rows, 1, inv_sqrt_d(g.D), ol);
    check_launch("qjl_dequant_kv_kernel");
    return true;
}

void launch_dequant(Scheme s, const uint8_t* pool, const int32_t* slots, uint16_t* out_key,
                    uint16_t* out_value, const PageGeom& g, int num_tokens, hipStream_t stream,
                    bool head_major) {
    const int rows = num_tokens * g.H;
    if (rows <= 0) return;
    const float inv = inv_sqrt_d(g.D);
    OutLayout ol;  // element offset of row (t, h): [N, H, D] or [H, N, D]
    ol.tok = head_major ? (uint64_t)g.D : (uint64_t)g.H * g.D;
    ol.head = head_major ? (uint64_t)num_tokens * g.D : (uint64_t)g.D;
    // D = 128 with 16-byte aligned codes: half a row per lane (2,048 waves
    // for a 32K-token, two-head layer: two per SIMD; 9.8 against 10.05 us for
    // the four-lanes-per-row kernel, 12.8 for a whole row per lane).
    if (rows <= kBufMaxRows && rows_dequant_ok(g, pool, out_key, out_value)) {
        constexpr int E1 = 64;
        const int rows_per_block = kBlock * E1 / 128;
        const int blocks_needed = (rows + rows_per_block - 1) / rows_per_block;
        const dim3 grid(std::max(1, std::min(blocks_needed, TQ_DEQ_ONE_BLOCKS_PER_CU * num_cus())));
        const LayerSet<1> one{{pool}, {out_key}, {out_value}};
        if (s == Scheme::Prod)
            hipLaunchKernelGGL((dequant_rows_kernel<1, 1, E1>), grid, dim3(kBlock), 0, stream, one,
                               slots, g, rows, 1, inv, ol);
        else
            hipLaunchKernelGGL((dequant_rows_kernel<0, 1, E1>), grid, dim3(kBlock), 0, stream, one,
                               slots, g, rows, 1, inv, ol);
        check_launch(s == Scheme::Prod ? "turbo_prod_dequant_kv_kernel" : "turbo_mse_dequant_kv_kernel");
        return;
    }
    if (wide_dequant_ok(g, pool, out_key, out_value)) {
        // Persistent waves: up to four workgroups (one wave per SIMD each) per
        // CU, fewer when there is not enough work (measured at D = 128: 4 per
        // CU beat 1 or 2 and equalled 8).
        const int rows_per_block = kBlock / (g.D / 32);
        const int blocks_needed = (rows + rows_per_block - 1) / rows_per_block;
        const dim3 grid(std::max(1, std::min(blocks_needed, TQ_DEQ_BLOCKS_PER_CU * num_cus())));
        const bool prod = s == Scheme::Prod;
        const LayerSet<1> one{{pool}, {out_key}, {out_value}};
        auto go = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, grid, dim3(kBlock), 0, stream, one, slots, g, rows, 1, inv,
                               ol);
        };
        if (g.D == 128) prod ? go(dequant_stream_kernel<128, 1>) : go(dequant_stream_kernel<128, 0>);
        else if (g.D == 64) prod ? go(dequant_stream_kernel<64, 1>) : go(dequant_stream_kernel<64, 0>);
        else prod ? go(dequant_stream_kernel<32, 1>) : go(dequant_stream_kernel<32, 0>);
        check_launch(prod ? "turbo_prod_dequant_kv_kernel" : "turbo_mse_dequant_kv_kernel");
        return;
    }
    const int rpb = kBlock / (g.D / 2);
    const dim3 grid((rows + rpb - 1) / rpb);
    if (s == Scheme::Prod) {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL((dequant_kernel<kD, true>), grid, dim3(kBlock), 0,
                                              stream, pool, slots, out_key, out_value, g, rows,
                                              inv, ol));
        check_launch("turbo_prod_dequant_kv_kernel");
    } else {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL((dequant_kernel<kD, false>), grid, dim3(kBlock), 0,
                                              stream, pool, slots, out_key, out_value, g, rows,
                                              inv, ol));
        check_launch("turbo_mse_dequant_kv_kernel");
    }
}

void launch_dequant_layers(Scheme s, const uint8_t* const* pools, const int32_t* slots,
                           uint16_t* const* out_key, uint16_t* const* out_value, const PageGeom& g,
                           int num_tokens, int num_layers, hipStream_t stream, bool head_major) {
    const int rows = num_tokens * g.H;
    if (rows <= 0 || num_layers <= 0) return;
    bool wide = g.D == 128;
    for (int l = 0; l < num_layers && wide; ++l)
        wide = wide_dequant_ok(g, pools[l], out_key[l], out_value[l]);
    if (!wide) {  // the per-layer kernels (other head dims, unaligned buffers)
        for (int l = 0; l < num_layers; ++l)
            launch_dequant(s, pools[l], slots, out_key[l], out_value[l], g, num_tokens, stream,
                           head_major);
        return;
    }
    const float inv = inv_sqrt_d(g.D);
    OutLayout ol;
    ol.tok = head_major ? (uint64_t)g.D : (uint64_t)g.H * g.D;
    ol.head = head_major ? (uint64_t)num_tokens * g.D : (uint64_t)g.D;
    const bool prod = s == Scheme::Prod;
    // A whole row per lane when every layer's buffers allow 16-byte code
    // loads (half a row per lane: 9.1 against 8.0 us per 32K-token layer).
    bool rows_ok = rows <= kBufMaxRows;
    for (int l = 0; l < num_layers && rows_ok; ++l)
        rows_ok = rows_dequant_ok(g, pools[l], out_key[l], out_value[l]);
    const int rows_per_block = rows_ok ? kBlock : kBlock / (g.D / 32);
    // The kernel counts (layer, row group) pairs in int32: keep them below 2^30.
    const int groups = (rows + 15) / 16;
    const int per_launch = (int)std::max(1LL, std::min<long long>(kMaxLayersPerLaunch,
                                                                  (1LL << 30) / groups));
    for (int l0 = 0; l0 < num_layers; l0 += per_launch) {
        const int n = std::min(per_launch, num_layers - l0);
        LayerSet<kMaxLayersPerLaunch> set{};
        for (int l = 0; l < n; ++l) {
            set.pool[l] = pools[l0 + l];
            set.out_key[l] = out_key[l0 + l];
            set.out_value[l] = out_value[l0 + l];
        }
        const long long blocks_needed =
            ((long long)rows * n + rows_per_block - 1) / rows_per_block;
        const int per_cu = rows_ok ? TQ_DEQ_ROWS_BLOCKS_PER_CU : TQ_DEQ_LAYERS_BLOCKS_PER_CU;
        const dim3 grid((unsigned)std::max(
            1LL, std::min<long long>(blocks_needed, (long long)per_cu * num_cus())));
        if (rows_ok) {
            if (prod)
                hipLaunchKernelGGL((dequant_rows_kernel<1, kMaxLayersPerLaunch, 128>), grid,
                                   dim3(kBlock), 0, stream, set, slots, g, rows, n, inv, ol);
            else
                hipLaunchKernelGGL((dequant_rows_kernel<0, kMaxLayersPerLaunch, 128>), grid,
                                   dim3(kBlock), 0, stream, set, slots, g, rows, n, inv, ol);
        } else if (prod)
            hipLaunchKernelGGL((dequant_stream_kernel<128, 1, kMaxLayersPerLaunch>), grid,
                               dim3(kBlock), 0, stream, set, slots, g, rows, n, inv, ol);
        else
            hipLaunchKernelGGL((dequant_stream_kernel<128, 0, kMaxLayersPerLaunch>), grid,
                               dim3(kBlock), 0, stream, set, slots, g, rows, n, inv, ol);
        check_launch(prod ? "turbo_prod_dequant_kv_layers" : "turbo_mse_dequant_kv_layers");
    }
}

}  // namespace tq

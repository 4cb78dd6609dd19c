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
#include <type_traits>

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

// Where the generic decode finds a row's tokens.  Slot-mapped rows all attend
// tokens [0, n) of one slot list (a negative slot: no token).
struct SlotTokens {
    const int32_t* slots;
    int n;
    struct Row {
        int kv;
    };
    __device__ Row row(int) const { return {n}; }
    __device__ bool cell(const Row&, int t, const PageGeom& g, int& page, int& tib) const {
        const int s = slots[t];
        if (s < 0) return false;
        split_slot(s, g, page, tib);
        return true;
    }
};
// Paged rows: query row q attends the first min(row_kv_len[q], max_kv_len)
// tokens of sequence row_seq[q]; token t is at position t % B of page
// block_tables[seq * max_blocks + t / B] (a negative page: no token).
// max_kv_len <= max_blocks * B (checked on the host) keeps t / B in the row.
struct PagedTokens {
    const int32_t* block_tables;
    const int32_t* row_seq;
    const int32_t* row_kv_len;
    int max_blocks, max_kv_len;
    struct Row {
        int kv, seq;
    };
    __device__ Row row(int q) const { return {min(row_kv_len[q], max_kv_len), row_seq[q]}; }
    __device__ bool cell(const Row& r, int t, const PageGeom& g, int& page, int& tib) const {
        const int blk = g.bs_shift >= 0 ? t >> g.bs_shift : t / g.block_size;
        page = block_tables[(size_t)r.seq * max_blocks + blk];
        tib = t - blk * g.block_size;
        return page >= 0;
    }
};

// ---------------------------------------------------------------------------
// Split-K partial: one wave per (split, row = q*H + h).
// ws[(split * rows + row) * (D + 2) + ...] = acc[0..D), m, l.
// Any head_dim and page geometry (the matrix-core kernels take D = 128 with
// aligned pages).
// ---------------------------------------------------------------------------
template <int D, bool PROD, class Tok>
__global__ __launch_bounds__(64) void attn_partial_kernel(
    const uint16_t* __restrict__ query, const uint8_t* __restrict__ pool, Tok tok,
    float* __restrict__ ws, PageGeom g, int rows, int tokens_per_split, int num_splits,
    float inv) {
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
    const typename Tok::Row tr = tok.row(row / g.H);

    float q0, q1;
    rotate_query<L>(query + (size_t)row * D, h, j, inv, q0, q1);

    const int t0 = split * tokens_per_split;
    const int t1 = min(tr.kv, t0 + tokens_per_split);
    float m = kInitMax, l = 0.0f, a0 = 0.0f, a1 = 0.0f;
    for (int t = t0; t < t1; ++t) {
        int page, tib;
        if (!tok.cell(tr, t, g, page, tib)) continue;  // no token here (wave-uniform)
        const CellPtrs c{pool + (size_t)page * g.page_size, (size_t)(tib * g.H + h)};
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
    if (slots[t] < 0) {  // unmapped token: excluded, like a -inf logit
        logits[(size_t)row * num_kv_tokens + t] = -INFINITY;
        return;
    }
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

// ===========================================================================
// Matrix-core path: D = 128, up to 8 query rows per kv head per workgroup.
//
// Per kv head h and row group (8 query rows), a workgroup of 4 waves owns a
// range of tokens; each wave takes 64-token chunks.
//   QK: S^T[token][col] = sum_d K[token][d] * Q^T[d][col] with
//       v_mfma_f32_16x16x32_f16.  A = K, decoded from nibbles to fp16 through
//       256-entry LDS tables indexed by code byte; B = the rotated query split
//       into fp16 hi + lo parts, columns 2r (hi) and 2r+1 (lo) of row r, so a
//       single MFMA column pair recovers ~22-bit query precision.  The K3
//       codebook enters as fp16(aK*K3[c]) with aK = 1.2918981, which makes all
//       four magnitudes fp16-exact to 1.4e-5 relative (V4 with aV = 1.5982153
//       to 9.3e-5); the scale is divided out per token.  turbo_prod's residual
//       sign is a second A matrix (+-1, exact) with its own accumulator.
//   softmax: base-2 online softmax per row over the chunk, in the MFMA output
//       layout (lane (col, g) holds tokens 4g..4g+3 of each 16-token tile).
//   PV: O[col][d] += sum_t P'[col][t] V[t][d] with the same MFMA.  The QK
//       output layout is exactly the A-operand layout over 32 tokens (two
//       tiles), so P' = p * vs needs no data movement; it is split hi/lo in
//       the column pair like q.  B = V, whose contraction index (tokens) must
//       run inside a lane: each lane loads dword i of 8 tokens' V cells and
//       interleaves the nibbles of token pairs into bytes, one table lookup
//       per (token pair, d).
// Each workgroup merges its waves, applies the inverse WHT and sign flip to
// its unnormalised partial (linear, so allowed before the split merge), and
// writes (o[128], m, l) per row; a combine kernel takes the weighted sum.
// ===========================================================================
namespace mfma {
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr float kAlphaK = 1.2918981f;
constexpr float kAlphaV = 1.5982153f;
// turbo_mse K: the fp16 table of aV*V4 alone is exact only to 9.2e-5, which
// logits of magnitude ~40 (outlier channels shared by q and k) turn into
// ~1e-3 output errors.  A second table holds the fp16 residual
// (aV*c - fp16(aV*c)) * 2^kLoShift per code, multiplied by the same query
// operand in its own accumulator and scaled back by 2^-kLoShift.
constexpr int kLoShift = 10;
constexpr float kLoScale = 1.0f / (float)(1 << kLoShift);
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kRows = 8;     // query rows per workgroup (16 MFMA columns, hi/lo)
// Page schemes of the split kernel: turbo_mse, turbo_prod, and the
// reference's unexported QJL-1b page (K = +-1 signs times one fp16 scale per
// (token, head); src/cuda/tq_qjl_kernels.cu).
constexpr int kSchMse = 0, kSchProd = 1, kSchQjl = 2;
constexpr int kPartStride = 128 + 4;  // floats per partial row: o[128], m, l, pad (16-B rows)

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    return __builtin_bit_cast(uint32_t, (half2v){(_Float16)a, (_Float16)b});
}
// (x - fp16(x)) * 2^kLoShift (exact in fp32), rounded to fp16 by pack_h2.
__device__ __forceinline__ float lo_part(float x) {
    return (x - (float)(_Float16)x) * (float)(1 << kLoShift);
}
// One 16x16x32 fp16 MFMA: c += a * b (fp32 accumulate).
__device__ __forceinline__ f32x4 mma(half8 a, half8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ half8 as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(half8, (u32x4){a, b, c, d});
}
// Batched decode over paged sequences: query row r belongs to sequence
// row_seq[r] (the 8 rows of an aligned group share one) and attends its
// first row_kv_len[r] tokens; token t of sequence s is in page
// block_tables[s * max_blocks + t / B].
// A unit: the npos consecutive row groups (new-token positions) of one
// sequence from row group `first` on, computed together.  It has one item
// per kv head; each item is n passes (workgroup-wide chunk steps of kPass
// tokens) over the unit's first kv_end tokens, a pass weighing w work units,
// at work positions [start, start + w*n) of its head's work (every head has
// the same work, split into segments per head).
struct PagedUnit {
    int32_t first, npos, kv_end, start, n, w, index, pad;  // index: the unit's number
};
struct PagedRows {
    const int32_t* block_tables;
    const int32_t* row_seq;
    const int32_t* row_kv_len;
    int max_blocks;
    // The step's plan (paged_plan_kernel): plan[0] units, then a sentinel
    // whose start is the total work plan[1]; a copy of each row group's unit.
    const PagedUnit* units;
    const PagedUnit* group_unit;
    const int32_t* plan;
    // A page-sized region of the workspace that masked tokens' loads address
    // (always valid memory; what they read is not used)
    const uint8_t* spare_page;
};
// Workgroup s of G takes the work positions [bound(s), bound(s + 1)) with
// bound(s) = floor(s * total / G) = q*s + floor(r*s / G) (q, r = total div, mod
// G; r*s < G*G stays in 32 bits); a pass belongs to the segment holding its
// first work position.
struct Segments {
    int q, r, G;
    __device__ Segments(int total, int g) : q(total / g), r(total % g), G(g) {}
    __device__ int bound(int s) const { return q * s + (int)((uint32_t)(r * s) / (uint32_t)G); }
    // The segment holding work position x < total: an estimate within one of
    // floor(((x + 1) G - 1) / total), then corrected.
    __device__ int of(int x, int total) const {
        int g = (int)(((float)x + 1.0f) * (float)G / (float)total) - 1;
        g = max(0, min(g, G - 1));
        while (g + 1 < G && bound(g + 1) <= x) ++g;
        while (g > 0 && bound(g) > x) --g;
        return g;
    }
};
// Passes [x0, x1) of an item (start S, n passes of weight w) that begin in
// the work range [b0, b1).
__device__ __forceinline__ void item_passes(int S, int n, int w, int b0, int b1, int& x0,
                                            int& x1) {
    x0 = S >= b0 ? 0 : (b0 - S + w - 1) / w;
    x1 = S >= b1 ? 0 : min(n, (b1 - S + w - 1) / w);
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS accesses,
// not for its outstanding global loads (which __syncthreads() would drain).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// fp16 hi or lo part of x: lo = fp16(x - fp32(fp16(x))) (the difference is exact).
__device__ __forceinline__ _Float16 hi_lo(float x, bool lo) {
    const _Float16 h = (_Float16)x;
    return lo ? (_Float16)(x - (float)h) : h;
}
// The lo parts of (x0, x1) as an fp16 pair, given their hi parts h (fp16
// pair, low half x0's): fp16(x - hi) with v_fma_mix (x * 1 - hi rounded once;
// the difference is exact in fp32), one instruction per half.
__device__ __forceinline__ uint32_t lo_pair(float x0, float x1, uint32_t h) {
    uint32_t r;
    asm("v_fma_mixlo_f16 %0, %1, 1.0, -%3 op_sel_hi:[0,0,1]\n\t"
        "v_fma_mixhi_f16 %0, %2, 1.0, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
        : "=&v"(r)
        : "v"(x0), "v"(x1), "v"(h));
    return r;
}
constexpr uint16_t f16_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
constexpr uint32_t f16_pair(float a, float b) {
    return (uint32_t)f16_bits(a) | ((uint32_t)f16_bits(b) << 16);
}
// (x - fp16(x)) * 2^kLoShift, exact in fp32 (mfma::lo_part at compile time).
constexpr float lo_part_c(float x) { return (x - (float)(_Float16)x) * (float)(1 << kLoShift); }

// fp16 bits of the codebook values the decode tables hold: aK*K3[j],
// aV*V4[j], and the lo parts (x - fp16(x)) * 2^kLoShift of aV*V4[j].
struct Fp16Tables {
    uint32_t k3[8], v4[16], v4lo[16];
};
constexpr Fp16Tables make_fp16_tables() {
    Fp16Tables t{};
    for (int j = 0; j < 8; ++j) t.k3[j] = f16_bits(kAlphaK * dev::kK3[j]);
    for (int j = 0; j < 16; ++j) {
        t.v4[j] = f16_bits(kAlphaV * dev::kV4[j]);
        t.v4lo[j] = f16_bits(lo_part_c(kAlphaV * dev::kV4[j]));
    }
    return t;
}
constexpr Fp16Tables kF16 = make_fp16_tables();
// The fp16 pair (t[j], t[j + 1]).
template <int N>
constexpr uint32_t f16_pair_of(const uint32_t (&t)[N], int j) {
    return t[j] | (t[j + 1] << 16);
}
// Selector of entry g < 4 of a 4-entry fp16 table held as two fp16 pairs:
// bytes 2g, 2g + 1, then zeros.
__device__ __forceinline__ uint32_t lut4_sel(int g) {
    return (uint32_t)(2 * g) | ((uint32_t)(2 * g + 1) << 8) | 0x0C0C0000u;
}
// t[4m + g] (in the low half) for the 4-entry slice m of t, g given by sel.
template <int N>
__device__ __forceinline__ uint32_t lut4(const uint32_t (&t)[N], int m, uint32_t sel) {
    return __builtin_amdgcn_perm(f16_pair_of(t, 4 * m + 2), f16_pair_of(t, 4 * m), sel);
}
// Decode tables in the one-address-two-pairs layout: S rows (256 B each,
// 32 copies of the entry in bytes 0..127) at byte 0 and K|V rows at byte
// kOffKV (K copies in bytes 0..127, turbo_prod's V copies in 128..255); entry
// b holds the fp16 pairs of code byte b (low nibble = even d):
//   K: turbo_prod (aK*K3[b & 7], aK*K3[(b >> 4) & 7]); turbo_mse the hi
//      parts fp16(aV*V4[b & 15]), fp16(aV*V4[b >> 4]) (its V lookups read them
//      too);
//   S: turbo_prod the residual signs (nibble bit 3 set: +1.0, else -1.0);
//      turbo_mse the lo parts of aV*V4;
//   V (turbo_prod): (aV*V4[b & 15], aV*V4[b >> 4]).
// Wave w of 8 writes rows 32w .. 32w + 31 of each table from registers (no
// memory traffic): with those rows one nibble of every entry is uniform
// across the wave and the other comes from a 4-entry fp16 table by v_perm.
//   S rows, and turbo_mse's K rows: store k < 4 writes row 32w + 8k + lane / 8,
//     copies 4q .. 4q + 3 (q = lane % 8): low nibble 8(k % 2) + lane / 8, high
//     nibble 2w + k / 2;
//   turbo_prod's K | V rows: store k < 8 writes row 32w + 4k + lane / 16, group
//     lane % 16 (K copies, then V copies): low nibble 4(k % 4) + lane / 16, high
//     nibble 2w + k / 4.
template <bool PROD>
struct TableWords {
    static constexpr int kR1Stores = PROD ? 8 : 4;
    uint32_t r0[4], r1[kR1Stores];
};
template <bool PROD>
__device__ __forceinline__ TableWords<PROD> decode_table_words(int w, int lane) {
    TableWords<PROD> tw;
    uint32_t(&r0)[4] = tw.r0;
    uint32_t(&r1)[TableWords<PROD>::kR1Stores] = tw.r1;
    {
        const int g4 = lane >> 4, g8 = lane >> 3;
        const uint32_t sel4 = lut4_sel(g4), sel8 = lut4_sel(g8 & 3);
        const bool hi8 = (g8 & 4) != 0;
        if constexpr (PROD) {
            const uint32_t sh = (w & 4) ? 0x3C000000u : 0xBC000000u;  // row bit 7 = w bit 2
#pragma unroll
            for (int k = 0; k < 4; ++k) r0[k] = ((k & 1) ? 0x3C00u : 0xBC00u) | sh;  // row bit 3
            const bool vq = (lane & 8) != 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t vpair =
                    lut4(kF16.v4, k & 3, sel4) | (kF16.v4[2 * w + (k >> 2)] << 16);
                const uint32_t kpair =
                    lut4(kF16.k3, k & 1, sel4) | (kF16.k3[(2 * w + (k >> 2)) & 7] << 16);
                r1[k] = vq ? vpair : kpair;
            }
        } else {
            uint32_t llo[2], vlo[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                llo[hh] = hi8 ? lut4(kF16.v4lo, 2 * hh + 1, sel8) : lut4(kF16.v4lo, 2 * hh, sel8);
                vlo[hh] = hi8 ? lut4(kF16.v4, 2 * hh + 1, sel8) : lut4(kF16.v4, 2 * hh, sel8);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                r0[k] = llo[k & 1] | (kF16.v4lo[2 * w + (k >> 1)] << 16);
                r1[k] = vlo[k & 1] | (kF16.v4[2 * w + (k >> 1)] << 16);
            }
        }
    }
    return tw;
}
template <bool PROD>
__device__ __forceinline__ void store_decode_tables(uint32_t* lut, int kv_words, int w, int lane,
                                                    const TableWords<PROD>& tw) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
        *reinterpret_cast<u32x4*>(&lut[(32 * w + 8 * k + (lane >> 3)) * 64 + 4 * (lane & 7)]) =
            (u32x4){tw.r0[k], tw.r0[k], tw.r0[k], tw.r0[k]};
#pragma unroll
    for (int k = 0; k < TableWords<PROD>::kR1Stores; ++k) {
        const int row = PROD ? 32 * w + 4 * k + (lane >> 4) : 32 * w + 8 * k + (lane >> 3);
        const int q = PROD ? lane & 15 : lane & 7;
        *reinterpret_cast<u32x4*>(&lut[kv_words + row * 64 + 4 * q]) =
            (u32x4){tw.r1[k], tw.r1[k], tw.r1[k], tw.r1[k]};
    }
}
}  // namespace mfma

// ---------------------------------------------------------------------------
// turbo_prod logits on the matrix cores (D = 128; :346-434, 628-648).
//
// Per (token, row): logit = ks (s1 + re s2) / sqrt(D), the reference's
// s1*ks + s2*ks*re, with s1 = sum_d q_d K3[c_d] and s2 = sum_d q_d u3_d
// (u3 = +-1: nibble bit 3).  Both are v_mfma_f32_16x16x32_f16 products
// A (16 tokens x 32 dims) x B (32 dims x 16 columns): column 2r + p holds
// query row r's fp16 hi (p = 0) or lo (p = 1) part, so a column pair sums to
// ~22-bit query precision.  For s1, A is K3[c] split the same way into two
// matrices, fp16(K3[c]) and fp16(K3[c] - fp16(K3[c])), both accumulated into
// one fp32 sum (the four hi/lo cross products: ~2^-22 relative); for s2, A is
// the +-1 matrix (exact).
//
// K3 is odd under c -> 7 - c (K3[7 - c] = -K3[c]), so K3[c] = +-mag[m] with
// mag = K3[4..7], m = (c ^ (c < 4 ? 3 : 0)) & 3 and the sign of bit 2.  The
// fp16 values come from v_perm over a 4-entry register table (low bytes of
// the 4 magnitudes in one dword, high bytes in another), selected by m, then
// the sign bit is xor'ed in; the +-1 matrix is 0x3C00 with the sign bit.
//
// A workgroup of 8 waves takes 128 tokens of one kv head and one group of up
// to 8 query rows; wave w takes tokens 16w .. 16w + 15 (one MFMA tile) and
// rotates query row w.  Lane (i, g) = (lane % 16, lane / 16)
// holds A rows of token i over dims 32g .. 32g + 31: the contraction runs
// over the dims in the order (block kk, lane group g, e) -> dim
// 32g + 8kk + e, so each lane's codes of a tile are one 16-byte load (code
// dword kk = block kk).  The MFMA output lane (n, g) holds tokens 4g .. 4g + 3
// of column n; its token scales come from lanes 16g + m (ks) and
// 16g + 4 + m (re) of its own 16-lane row by DPP row broadcast.
// ---------------------------------------------------------------------------
namespace lgt {
using namespace mfma;
constexpr int kWaves = 8, kTilesW = 1, kTile = 16;  // 4.9 us/layer at 32K; 4 x 2: 5.2, 8 x 2: 5.1
constexpr int kTokens = kWaves * kTilesW * kTile;  // tokens per workgroup
constexpr uint16_t f16b(double x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
constexpr double f16v(double x) { return (double)(_Float16)x; }
constexpr double kmag(int m) { return (double)dev::kK3[4 + m]; }
constexpr uint16_t mag_hi(int m) { return f16b(kmag(m)); }
constexpr uint16_t mag_lo(int m) { return f16b(kmag(m) - f16v(kmag(m))); }
constexpr uint32_t bytes4(uint16_t a, uint16_t b, uint16_t c, uint16_t d, int hi_byte) {
    const int sh = 8 * hi_byte;
    return ((uint32_t)((a >> sh) & 0xFF)) | ((uint32_t)((b >> sh) & 0xFF) << 8) |
           ((uint32_t)((c >> sh) & 0xFF) << 16) | ((uint32_t)((d >> sh) & 0xFF) << 24);
}
// v_perm tables: byte m of the *L word is the low byte of magnitude m's
// fp16 value, byte m of the *H word its high byte.
constexpr uint32_t kHiL = bytes4(mag_hi(0), mag_hi(1), mag_hi(2), mag_hi(3), 0);
constexpr uint32_t kHiH = bytes4(mag_hi(0), mag_hi(1), mag_hi(2), mag_hi(3), 1);
constexpr uint32_t kLoL = bytes4(mag_lo(0), mag_lo(1), mag_lo(2), mag_lo(3), 0);
constexpr uint32_t kLoH = bytes4(mag_lo(0), mag_lo(1), mag_lo(2), mag_lo(3), 1);

// The three A operands of one code dword W (dims of byte k: low nibble ->
// low half of dword k, high nibble -> high half).
struct AOps {
    half8 hi, lo, u3;
};
__device__ __forceinline__ AOps a_ops(uint32_t W, uint32_t hil, uint32_t hih, uint32_t lol,
                                      uint32_t loh) {
    const uint32_t V = ~W;
    const uint32_t t = (V >> 2) & 0x11111111u;                    // 1 where c < 4
    const uint32_t wm = (W ^ (t | (t << 1))) & 0x33333333u;       // m per nibble
    const uint32_t E = wm & 0x03030303u, O = (wm >> 4) & 0x03030303u;
    const uint32_t xs = (V << 5) & 0x80808080u, ys = (V << 1) & 0x80808080u;  // K3 < 0
    const uint32_t x3 = ((V << 4) & 0x80808080u) | 0x3C3C3C3Cu;   // u3 of low nibbles
    const uint32_t y3 = (V & 0x80808080u) | 0x3C3C3C3Cu;          // of high nibbles
    uint32_t h[4], l[4], u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t sel =
            __builtin_amdgcn_perm(O, E, (uint32_t)(k | k << 8 | (4 + k) << 16 | (4 + k) << 24)) |
            0x04000400u;
        const uint32_t sk = (uint32_t)(0x0C | k << 8 | 0x0C << 16 | (4 + k) << 24);
        const uint32_t sg = __builtin_amdgcn_perm(ys, xs, sk);
        h[k] = __builtin_amdgcn_perm(hih, hil, sel) ^ sg;
        l[k] = __builtin_amdgcn_perm(loh, lol, sel) ^ sg;
        u[k] = __builtin_amdgcn_perm(y3, x3, sk);
    }
    return {as_h8(h[0], h[1], h[2], h[3]), as_h8(l[0], l[1], l[2], l[3]),
            as_h8(u[0], u[1], u[2], u[3])};
}

template <int N>
__device__ __forceinline__ float row_bcast(float v) {  // lane N of each 16-lane row
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + N, 0xF, 0xF,
                                                      false));
}
template <int N>
__device__ __forceinline__ int row_bcast_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x150 + N, 0xF, 0xF, false);
}

// VEC: the logits rows are 16-byte aligned and num_kv_tokens % 4 == 0.
template <bool VEC>
__global__ __launch_bounds__(64 * kWaves) void prod_logits_mfma_kernel(
    const uint16_t* __restrict__ query, const uint8_t* __restrict__ pool,
    const int32_t* __restrict__ slots, float* __restrict__ logits, PageGeom g, int num_queries,
    int num_kv_tokens, float inv) {
    constexpr int D = 128;
    __shared__ uint32_t bq[4][64][4];  // B operands: [block kk][lane][dword], fp16 pairs
    // Every kernel argument the loads need, fetched in the first batch of
    // scalar loads (one wait) rather than each before its first use.
    asm volatile("" ::"s"(pool), "s"(slots), "s"(logits), "s"(g.page_size), "s"(g.kc_off),
                 "s"(g.ks_off), "s"(g.kres_off), "s"(g.H), "s"(g.bs_shift));
    const int h = blockIdx.y, rg = blockIdx.z;
    const int nrows = min(kRows, num_queries - rg * kRows);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int i = lane & 15, gq = lane >> 4;
    const int t0 = blockIdx.x * kTokens + w * (kTilesW * kTile);
    // Loads first, in dependency order: the wave's two query rows (raw), the
    // slots of the lane's code token (i) and scale token (4 gq + lane % 4) of
    // each tile, then the codes and the one scale (ks for lane % 8 < 4, else
    // re).  Dropped tokens read the query's first bytes (always valid
    // memory); their addresses are selected, then hidden from the optimiser
    // so each value stays one unconditional load.
    constexpr int kRowsW = kRows / kWaves;  // query rows rotated per wave
    uint32_t qq[kRowsW];
#pragma unroll
    for (int e = 0; e < kRowsW; ++e) {
        const int r = w + kWaves * e;
        qq[e] = r < nrows ? *reinterpret_cast<const uint32_t*>(
                                query + ((size_t)(rg * kRows + r) * g.H + h) * D + 2 * lane)
                          : 0u;
    }
    int slot_c[kTilesW], slot_s[kTilesW];
#pragma unroll
    for (int tt = 0; tt < kTilesW; ++tt) {
        const int tc = t0 + kTile * tt + i, ts = t0 + kTile * tt + 4 * gq + (lane & 3);
        slot_c[tt] = tc < num_kv_tokens ? slots[tc] : -1;
        slot_s[tt] = ts < num_kv_tokens ? slots[ts] : -1;
    }
    const uint64_t dummy = reinterpret_cast<uint64_t>(query);
    const uint64_t soff = (lane & 4) ? g.kres_off : g.ks_off;
    typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
    u32x4 code[kTilesW];
    uint16_t sraw[kTilesW];
#pragma unroll
    for (int tt = 0; tt < kTilesW; ++tt) {
        int page, tib;
        split_slot(slot_c[tt] >= 0 ? slot_c[tt] : 0, g, page, tib);
        // (page sizes are below 4 GiB: checked by the launcher)
        uint64_t ac = slot_c[tt] >= 0
                          ? reinterpret_cast<uint64_t>(pool) +
                                (uint64_t)(uint32_t)page * (uint32_t)g.page_size + g.kc_off +
                                (uint32_t)((tib * g.H + h) * g.code_stride + 16 * gq)
                          : dummy;
        split_slot(slot_s[tt] >= 0 ? slot_s[tt] : 0, g, page, tib);
        uint64_t as = slot_s[tt] >= 0
                          ? reinterpret_cast<uint64_t>(pool) +
                                (uint64_t)(uint32_t)page * (uint32_t)g.page_size + soff +
                                (uint32_t)((tib * g.H + h) * g.scale_stride)
                          : dummy;
        asm volatile("" : "+v"(ac), "+v"(as));
        // 16 code bytes at a 4-byte aligned address (one multi-dword load;
        // global loads need dword alignment only).
        code[tt] = *reinterpret_cast<const __attribute__((address_space(1))) u32x4a4*>(ac);
        sraw[tt] = *reinterpret_cast<const __attribute__((address_space(1))) uint16_t*>(as);
    }

    // Rotate the wave's query rows w + 8e / kWaves (sign flip, orthonormal
    // WHT) while the codes load; lane j holds dims 2j, 2j + 1: block kk = (j % 16) / 4, lane group
    // g = j / 16, dword j % 4 of columns 2r (hi) and 2r + 1 (lo).
    {
        const float sh = (h & 1) ? -1.0f : 1.0f;
        const int kk = (lane & 15) >> 2, cg = 16 * (lane >> 4);
#pragma unroll
        for (int e = 0; e < kRowsW; ++e) {
            float q0 = h2f(qq[e] & 0xffff) * sh, q1 = h2f(qq[e] >> 16) * (-sh);
            wht_pair<D / 2>(q0, q1, lane);
            q0 *= inv;
            q1 *= inv;
            const uint32_t hi = pack_h2(q0, q1);
            const int col = 2 * (w + kWaves * e) + cg;
            bq[kk][col][lane & 3] = hi;
            bq[kk][col + 1][lane & 3] = lo_pair(q0, q1, hi);
        }
    }
    // Register tables for the K operands (values in VGPRs: v_perm reads at
    // most one scalar operand).
    uint32_t hil = kHiL, hih = kHiH, lol = kLoL, loh = kLoH;
    asm volatile("" : "+v"(hil), "+v"(hih), "+v"(lol), "+v"(loh));
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    half8 b[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
        b[kk] = __builtin_bit_cast(half8, *reinterpret_cast<const u32x4*>(bq[kk][lane]));

    const int r = i >> 1;
    const bool writer = (i & 1) == 0 && r < nrows;
    float* const row_out = logits + ((size_t)(rg * kRows + r) * g.H + h) * num_kv_tokens;
#pragma unroll
    for (int tt = 0; tt < kTilesW; ++tt) {
        f32x4 s1 = {0.f, 0.f, 0.f, 0.f}, s2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const AOps a = a_ops(code[tt][kk], hil, hih, lol, loh);
            s1 = mma(a.hi, b[kk], s1);
            s2 = mma(a.u3, b[kk], s2);
            s1 = mma(a.lo, b[kk], s1);
        }
        // Lane (n, gq): tokens 4 gq + m of column n; rows r = n / 2 summed
        // over the hi/lo column pair, then scaled by the token's ks.
        const float sv = h2f(sraw[tt]);
        const float ksm[4] = {row_bcast<0>(sv), row_bcast<1>(sv), row_bcast<2>(sv),
                              row_bcast<3>(sv)};
        const float rem[4] = {row_bcast<4>(sv), row_bcast<5>(sv), row_bcast<6>(sv),
                              row_bcast<7>(sv)};
        const int okm[4] = {row_bcast_i<0>(slot_s[tt]), row_bcast_i<1>(slot_s[tt]),
                            row_bcast_i<2>(slot_s[tt]), row_bcast_i<3>(slot_s[tt])};
        float out[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            float x = s1[m] + rem[m] * s2[m];
            x += lane_xor<1>(x);
            out[m] = okm[m] < 0 ? -INFINITY : x * ksm[m] * inv;
        }
        const int tf = t0 + kTile * tt + 4 * gq;
        if (writer) {
            float* dst = row_out + tf;
            if (VEC && tf + 3 < num_kv_tokens) {
                *reinterpret_cast<float4*>(dst) = make_float4(out[0], out[1], out[2], out[3]);
            } else {
#pragma unroll
                for (int m = 0; m < 4; ++m)
                    if (tf + m < num_kv_tokens) dst[m] = out[m];
            }
        }
    }
}
}  // namespace lgt

// CH = tokens per wave iteration (32: two QK tiles, one PV step; 64: four and
// two); NW = waves per workgroup; NP = row groups per workgroup.
// NP = 1: the 16 MFMA columns are the group's 8 query rows as fp16 hi and lo
// parts (columns 2r, 2r + 1), summed after each product.
// NP = 2 or 4 (paged rows): the new tokens (row groups) of one sequence in a
// unit share every decoded K/V chunk; each tile of 16 columns is (position,
// row) = (i / 8, i % 8) of two positions, and the hi and lo parts are stacked
// along the reduction instead (QK: the same decoded K against the hi and the
// lo query; PV: the hi and the lo P against the same decoded V), so each
// lane's column is one query row and its softmax runs once.  A unit of one
// position uses the one-group column layout in its tile.  PAGED: the grid is
// one workgroup per work segment of the step's plan (paged_plan_kernel).
// SCH = page scheme (kSch*).  QJL: the A operand of QK is the +-1 sign
// matrix, read as fp16 octets from an LDS table indexed by sign byte; the
// logit is ks * <qrot, signs> (no 1/sqrt(D) beyond the rotation's, :254);
// the rotation's sign flip has no head term.
template <int SCH, int CH, int NW, bool PAGED, int NP = 1>
__global__ __launch_bounds__(64 * NW) void attn_mfma_split_kernel(
    const uint16_t* __restrict__ query, const uint8_t* __restrict__ pool,
    const int32_t* __restrict__ slots, float* __restrict__ ws, float inv, int num_queries,
    int num_kv_tokens, int tokens_per_split, int num_splits, PageGeom g, mfma::PagedRows pr) {
    using namespace mfma;
    constexpr int kChunk = CH, kWaves = NW;
    constexpr int kTiles = CH / 16, kSteps = CH / 32;
    static_assert(CH == 32 || CH == 64, "chunk of 32 or 64 tokens");
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    static_assert(NP == 1 || ((NP == 2 || NP == 4) && PAGED), "2 or 4 positions: paged rows");
    constexpr bool PROD = SCH == kSchProd, QJL = SCH == kSchQjl;
    static_assert(!QJL || (!PAGED && NP == 1), "QJL: slot-mapped rows, one position");
    constexpr int kR = kRows * NP;  // query rows of the workgroup
    // NP >= 2: NT tiles of 16 MFMA columns, (position 2t + i / 8, row i % 8)
    constexpr int NT = NP >= 2 ? NP / 2 : 1;
    constexpr int kMoRows = NP >= 2 ? 16 : kR;  // rows merged per pass (one tile)
    // Decode tables indexed by a code byte (low nibble = even d), fp16 pairs,
    // 32 copies each: copy c of entry e at byte 256e + 4c of its table and lane
    // l reads copy l % 32, so a half-wave's 32 random lookups hit 32 distinct
    // banks.
    //  - NP = 1 (the QJL-1b decode; the layout the one-group loop reads for
    //    any scheme): one region of K|V rows, table 0 in bytes 0..127 of each
    //    row (QJL: the sign octets; prod: aK*K3; mse: the lo parts of aV*V4)
    //    and table 1 = V (aV*V4) in bytes 128..255.
    //  - NP >= 2 (turbo_prod, turbo_mse): the layout of decode_table_words,
    //    S rows at byte 0 and K|V rows at byte kOffKV.  One address then reads
    //    a code byte's S pair (offset 0) and its K pair (offset kOffKV, which
    //    no two-address LDS read merges with 0), each straight into its MFMA
    //    operand, and a V lookup's address is that of the byte's S row + 128
    //    (turbo_prod's V copies; turbo_mse reads its K copies, + 0).
    // After the token loop the tables' space holds the per-wave results for
    // the merge (NP = 1: the K|V rows; NP >= 2: one tile in each half).
    constexpr bool STAB = NP >= 2;
    constexpr int kOffKV = STAB ? 65520 : 0;
    constexpr int kTabWords = STAB ? 32768 : 256 * 64;
    __shared__ __attribute__((aligned(256))) uint32_t lut[kTabWords];
    __shared__ float qs_sep[STAB ? 1 : kR][128];  // NP = 1: the rotated queries
    __shared__ uint4 bqs[NP][4][64];  // QK B operand (fp16 hi/lo q) of k-step s for lane l
    __shared__ uint64_t tko[kWaves][kChunk], tvo[kWaves][kChunk];
    __shared__ float4 tsc[kWaves][kChunk];  // per token: K scale a, residual scale b, vs, bias
    __shared__ float mm[kWaves][kR], ml[kWaves][kR];
    __shared__ uint32_t kstage[256], vstage[256];  // NP = 1: the staged table entries
    static_assert(kOffKV + 256 * 256 <= (int)sizeof(lut), "K|V rows");
    static_assert(kOffKV + sizeof(float) * kWaves * kMoRows * 128 <= sizeof(lut), "merge space");
    float(*mo)[kMoRows][128] = reinterpret_cast<float(*)[kMoRows][128]>(&lut[kOffKV / 4]);
    // K|V row e (its 64 words: 32 K copies, then 32 V copies)
    auto kv_row = [&](int e) -> uint32_t* { return &lut[kOffKV / 4 + 64 * e]; };
    // Rotated query element (r, d) (NP = 1; NP >= 2 writes the B operands
    // directly)
    auto qs_at = [&](int r, int d) -> float& { return qs_sep[STAB ? 0 : r][d]; };

    // logit scale per unit ks (log2(e) / alpha folded at compile time: no run-time division)
    const float ck = inv * (PROD ? kLog2e / kAlphaK : kLog2e / kAlphaV);
    const float cr = inv * kLog2e;                                 // residual: ks * re
    // One work item: kv head h, row groups rg .. rg + npos - 1, tokens
    // [t_begin, t_cap) (paged: and below each row's length), partial slot pid.
    // (tid is a parameter so that a caller looping over items can keep the
    // per-thread values derived from it from being hoisted out of the loop
    // and held across the token loop.)
    auto item = [&](const int tid, const int h, const int rg, const int npos, const int t_begin,
                    const int t_cap, const size_t pid) {
        const int lane = tid & 63;
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
        const int i = lane & 15, gq = lane >> 4;
        // Paged rows: the group's sequence and per-row kv lengths (causal limit);
        // rowlen is that of this lane's MFMA column row.  A piece past every row's
        // length has no partial (the combine does not read it).
        int kv_end = num_kv_tokens, seq = 0;
        // per position: this lane's column row length, the group's longest and
        // shortest row
        int rowlen[NP] = {}, gend[NP] = {}, gmin[NP] = {};
        // NP >= 2: this lane's column row length per tile and the shortest live row
        int rl_col[NT] = {}, gmin_live = 0x7fffffff;
        // This wave's query rows (row r of the workgroup is row r % 8 of group
        // rg + r / 8: rows rg * 8 + r), loaded before anything waits: paged rows
        // issue them right after the row lengths and the sequence, so the
        // length processing waits only for those (the vector-memory counter is
        // in order) while the queries are in flight.
        constexpr int kQPerWave = kR / kWaves;
        static_assert(kR % kWaves == 0, "rows per wave");
        uint32_t qraw[kQPerWave];
        auto load_queries = [&]() {
#pragma unroll
            for (int k = 0; k < kQPerWave; ++k) {
                const int qi = min(rg * kRows + w + k * kWaves, num_queries - 1);
                qraw[k] = *reinterpret_cast<const uint32_t*>(query + ((size_t)qi * g.H + h) * 128 +
                                                              2 * lane);
            }
        };
        if constexpr (!PAGED) load_queries();
        if constexpr (PAGED) {
            kv_end = 0;
            // Every row length and the sequence are loaded unconditionally (rows
            // past the end re-read the last row), so the loads go out together:
            // a load under a condition sits in a branch whose join waits for it.
            int lraw[NP];
#pragma unroll
            for (int p = 0; p < NP; ++p)
                lraw[p] = pr.row_kv_len[min((rg + p) * kRows + (lane & 7), num_queries - 1)];
            const int seq_raw = pr.row_seq[rg * kRows];
            load_queries();
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const int rr = (rg + p) * kRows + (lane & 7);
                const int lv = p < npos && rr < num_queries ? lraw[p] : 0;
                rowlen[p] = __shfl(lv, i >> 1);
                const int lc = __shfl(lv, i & 7);
                // (one position: both halves of the tile hold its rows, hi and lo)
                if (NP >= 2 && (npos == 1 ? p == 0 : (i >> 3) == (p & 1))) rl_col[p >> 1] = lc;
                int m = max(lv, __shfl_xor(lv, 1)), n = min(lv, __shfl_xor(lv, 1));
                m = max(m, __shfl_xor(m, 2));
                n = min(n, __shfl_xor(n, 2));
                m = max(m, __shfl_xor(m, 4));
                n = min(n, __shfl_xor(n, 4));
                gend[p] = __builtin_amdgcn_readfirstlane(m);
                gmin[p] = __builtin_amdgcn_readfirstlane(n);
                kv_end = max(kv_end, gend[p]);
                if (p < npos) gmin_live = min(gmin_live, gmin[p]);
            }
            seq = __builtin_amdgcn_readfirstlane(seq_raw);
            // (a piece always starts below its unit's kv end: the walk calls
            // this only for work positions below ceil(kv_end / pass); a piece
            // past every row would run no chunk and write no partial)
        }
        const int t_end = min(kv_end, t_cap);
        const int ntile = (npos + 1) >> 1;  // NP >= 2: tiles of 16 columns in use

        // A chunk's codes and per-token scales, loaded ahead of its compute.
        struct Chunk {
            uint4 kw[kTiles];        // K: tile tau, token 16*tau + i, bytes [16gq, 16gq + 16)
            uint32_t vw[kSteps][8];  // V: step p, k-index 8gq + e (token below), dword i
            uint16_t ks, re, vs;  // this lane's token's fp16 scales (raw: still in flight)
            bool valid;
        };
        // Token of this lane in the chunk at t0 (lanes past the range re-read the
        // last token of the range) and its slot, or for paged rows its page
        // table entry.  The load is issued here and consumed by fetch, so other
        // work runs in between; arithmetic on the loaded value here would make
        // the in-order vector-memory counter wait, right after the next chunk's
        // code loads are issued, for all of them (129-130 -> 125-127.5 us per
        // config-5 step).
        auto chunk_token = [&](int t0) -> int {
            return max(min(t0 + (lane & (kChunk - 1)), t_end - 1), 0);
        };
        auto load_slot = [&](int t0) -> int {
            const int t = chunk_token(t0);
            if constexpr (PAGED) {  // token t of sequence seq: page table entry t / B
                const int blk = g.bs_shift >= 0 ? t >> g.bs_shift : t / g.block_size;
                return pr.block_tables[(size_t)seq * pr.max_blocks + min(blk, pr.max_blocks - 1)];
            } else {
                return slots[t];
            }
        };
        // slot -> cell offsets (exchanged through LDS) -> scale and code loads,
        // issued for every lane.  Slot-mapped rows: tokens past the range or
        // with a negative slot read the first bytes of the query instead (always
        // valid memory: the offset of the query from the pool) and get bias
        // -inf.  The loads stay in flight until the chunk is computed.
        const uint64_t dummy_off =
            (uint64_t)(reinterpret_cast<uintptr_t>(query) - reinterpret_cast<uintptr_t>(pool));
        // Slot-mapped rows read each pool byte once: non-temporal loads keep
        // the L2 for the slots and queries (10.3 -> 10.0 us per 32K layer).
        // Paged rows keep plain loads: the workgroups of the two kv heads of
        // a work segment read each 128-byte code line together, one through
        // the other's L2 copy.
        typedef __attribute__((address_space(1))) const uint8_t gbyte;
        typedef __attribute__((address_space(1))) const uint32_t gword;
        typedef __attribute__((address_space(1))) const u32x4 gquad;
        auto ld16 = [](const uint8_t* p) -> uint16_t { return PAGED ? ld_u16(p) : ld_u16_nt(p); };
        auto ld32 = [](gbyte* p) -> uint32_t {
            if constexpr (PAGED) return *reinterpret_cast<gword*>(p);
            return ld_u32_nt((const uint8_t*)p);
        };
        auto ld128 = [](gbyte* p) -> uint4 {
            if constexpr (PAGED) return __builtin_bit_cast(uint4, *reinterpret_cast<gquad*>(p));
            return ld_u4_nt((const uint8_t*)p);
        };
        // The code rows' addresses go through LDS: paged rows as global
        // addresses, slot-mapped rows as offsets from pool.
        auto code_row = [&](uint64_t v) -> gbyte* {
            return PAGED ? reinterpret_cast<gbyte*>(v) : (gbyte*)(pool + v);
        };
        auto fetch = [&](int t0, int loaded, Chunk& c) {
            if constexpr (PAGED) {
                // loaded: the token's page table entry.  A cell's bytes are its
                // page's address plus 32-bit offsets within the page (integer
                // selects: no branches around loads).  Masked lanes (past the
                // range, or an unmapped page) address the workspace's spare page
                // instead: always valid memory, its bytes unused (bias -inf).
                c.valid = t0 + (lane & (kChunk - 1)) < t_end && loaded >= 0;
                const int t = chunk_token(t0);
                const int tib = g.bs_shift >= 0 ? t & (g.block_size - 1) : t % g.block_size;
                const uint32_t cell = (uint32_t)(tib * g.H + h);
                const uint8_t* pg =
                    c.valid ? pool + (uint64_t)(uint32_t)loaded * (uint32_t)g.page_size
                            : pr.spare_page;
                const uint32_t so = cell * (uint32_t)g.scale_stride;
                c.ks = ld16(pg + (so + (uint32_t)g.ks_off));
                c.vs = ld16(pg + (so + (uint32_t)g.vs_off));
                c.re = PROD ? ld16(pg + (so + (uint32_t)g.kres_off)) : (uint16_t)0;
                const uint32_t co = cell * (uint32_t)g.code_stride;
                tko[w][lane & (kChunk - 1)] = reinterpret_cast<uint64_t>(pg + (co + (uint32_t)g.kc_off));
                tvo[w][lane & (kChunk - 1)] = reinterpret_cast<uint64_t>(pg + (co + (uint32_t)g.vc_off));
            } else {
                const int slot = loaded;
                c.valid = t0 + (lane & (kChunk - 1)) < t_end && slot >= 0;
                int page, tib;
                split_slot(c.valid ? slot : 0, g, page, tib);
                const uint64_t cell = (uint64_t)(tib * g.H + h);
                const uint64_t pb = (uint64_t)page * g.page_size;
                // Byte offsets from pool (integer selects: no branches around loads).
                // (distinct dummy bytes per field, so the three loads stay separate)
                const uint64_t so = pb + cell * g.scale_stride;
                c.ks = ld16(pool + (c.valid ? so + g.ks_off : dummy_off));
                c.vs = ld16(pool + (c.valid ? so + g.vs_off : dummy_off + 2));
                c.re = PROD ? ld16(pool + (c.valid ? so + g.kres_off : dummy_off + 4)) : (uint16_t)0;
                // (with 32-token chunks lanes l and l + 32 hold the same token)
                // K row: code_stride bytes, or QJL's D/8 = 16 sign bytes
                const uint64_t kstride = QJL ? 16u : (uint64_t)g.code_stride;
                tko[w][lane & (kChunk - 1)] = c.valid ? pb + g.kc_off + cell * kstride : dummy_off;
                tvo[w][lane & (kChunk - 1)] =
                    c.valid ? pb + g.vc_off + cell * g.code_stride : dummy_off;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int tau = 0; tau < kTiles; ++tau) {
                if constexpr (QJL)  // sign bytes 4gq .. 4gq + 3: k-steps 0 .. 3
                    c.kw[tau] = make_uint4(
                        *reinterpret_cast<gword*>(code_row(tko[w][16 * tau + i]) + 4 * gq),
                        0u,
                        0u, 0u);
                else
                    c.kw[tau] = ld128(code_row(tko[w][16 * tau + i]) + 16 * gq);
            }
            // (the K words first: the QK waits for them while the V words may
            // still be in flight)
            __builtin_amdgcn_sched_barrier(0);
            // k-step p covers tiles 2p, 2p+1; k-index 8gq + e is token
            // 32p + 4gq + e (e < 4) or 32p + 16 + 4gq + (e - 4).
#pragma unroll
            for (int p = 0; p < kSteps; ++p)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int tok = 32 * p + (e < 4 ? 4 * gq + e : 16 + 4 * gq + (e - 4));
                    c.vw[p][e] = ld32(code_row(tvo[w][tok]) + 4 * i);
                }
        };

        // Issue order matters (the vector-memory counter is in order): the
        // query rows (above), then the first chunk's slots; the decode tables
        // are built while they are in flight.
        int t0 = t_begin + w * kChunk;
        const int slot0 = load_slot(t0);

        // NP = 1: decode tables staged one entry per thread (waves 0-3), then
        // replicated after the first barrier.
        if (!STAB && w < 4) {
            const int lo = tid & 15, hi = tid >> 4;
            const float vlo = pick(kV4, lo), vhi = pick(kV4, hi);
            const uint32_t vv = pack_h2(kAlphaV * vlo, kAlphaV * vhi);
            // prod: aK * K3; mse: the lo parts of aV * V4 (its hi parts are the V table)
            const uint32_t kv =
                PROD ? pack_h2(kAlphaK * pick(kK3, lo & 7), kAlphaK * pick(kK3, hi & 7))
                     : pack_h2(lo_part(kAlphaV * vlo), lo_part(kAlphaV * vhi));
            kstage[tid] = kv;
            vstage[tid] = vv;
        }
        // Query halves to fp32 (times the sign flip) before the code loads are
        // issued, so waiting for them never waits for the codes.
        float qf[kQPerWave][2];
        {
            const float sh = (!QJL && (h & 1)) ? -1.0f : 1.0f;
#pragma unroll
            for (int k = 0; k < kQPerWave; ++k) {
                qf[k][0] = h2f(qraw[k] & 0xffff) * sh;
                qf[k][1] = h2f(qraw[k] >> 16) * (-sh);
            }
        }
        Chunk cur;
        fetch(t0, slot0, cur);  // in flight during the setup below (empty waves: all invalid)

        const bool lo_col = (i & 1) != 0;  // NP = 1: column i holds row i / 2's hi (even) or lo part
        if constexpr (STAB) {
            static_assert(kWaves == 8 && kRows == 8, "eight waves, one row per wave and position");
            __builtin_amdgcn_sched_barrier(0);  // the first chunk's loads go out before the setup
            // The decode tables from registers, and each wave's rotated rows
            // (position k: row w of group rg + k) as fp16 hi and lo parts
            // straight into the QK B operand: one barrier for the setup.  Lane l
            // holds d = 2l, 2l + 1: k-group l / 16, k-step (l / 4) % 4, halves
            // 2(l % 4), + 1 of the half8.  Two or more positions: tile k / 2,
            // column 8(k % 2) + w, hi in operand 2(k / 2), lo in 2(k / 2) + 1;
            // one position: tile 0, hi in column w, lo in column w + 8.
            const TableWords<PROD> tw = decode_table_words<PROD>(w, lane);
            const int s_l = (lane >> 2) & 3, g_l = lane >> 4;
#pragma unroll
            for (int k = 0; k < kQPerWave; ++k) {
                if (k >= 2 * ntile || (npos == 1 && k > 0)) continue;  // never read (wave-uniform)
                float q0 = qf[k][0], q1 = qf[k][1];
                wht_pair<64>(q0, q1, lane);
                const bool live = k < npos && rg * kRows + w + k * kWaves < num_queries;
                q0 = live ? q0 * inv : 0.0f;
                q1 = live ? q1 * inv : 0.0f;
                const uint32_t hi = pack_h2(q0, q1);
                const uint32_t lo = lo_pair(q0, q1, hi);
                const int col_hi = npos == 1 ? w : 8 * (k & 1) + w;
                const int col_lo = npos == 1 ? w + 8 : col_hi;
                const int op_hi = npos == 1 ? 0 : 2 * (k >> 1);
                const int op_lo = npos == 1 ? 0 : op_hi + 1;
                reinterpret_cast<uint32_t*>(&bqs[op_hi][s_l][16 * g_l + col_hi])[lane & 3] = hi;
                reinterpret_cast<uint32_t*>(&bqs[op_lo][s_l][16 * g_l + col_lo])[lane & 3] = lo;
            }
            store_decode_tables<PROD>(lut, kOffKV / 4, w, lane, tw);
        } else {
        // Rotated query rows of this group (wave w: rows w, w + NW, ...):
        // qrot = WHT(q * s) * inv.
#pragma unroll
        for (int k = 0; k < kQPerWave; ++k) {
            const int r = w + k * kWaves;
            if (NP >= 2 && r / kRows >= 2 * ntile) continue;  // an unused tile (wave-uniform)
            float q0 = qf[k][0], q1 = qf[k][1];
            wht_pair<64>(q0, q1, lane);
            const bool live = r / kRows < npos && rg * kRows + r < num_queries;
            qs_at(r, 2 * lane) = live ? q0 * inv : 0.0f;
            qs_at(r, 2 * lane + 1) = live ? q1 * inv : 0.0f;
        }
        lds_barrier();  // staged table rows and rotated queries visible

        // Every wave replicates staged rows with conflict-free 1 KB stores.
        {
            constexpr int kRowsPerWave = 256 / kWaves;
            // (all staged words read before the first store: one LDS round trip)
            uint32_t stv[kRowsPerWave / 4];
            if constexpr (!QJL) {
#pragma unroll
                for (int k = 0; k < kRowsPerWave; k += 4) {
                    const int e = w * kRowsPerWave + k + (lane >> 4);
                    stv[k / 4] = (lane & 8) ? vstage[e] : kstage[e];  // words 32..63: V
                }
            }
#pragma unroll
            for (int k = 0; k < kRowsPerWave; k += 4) {
                const int e = w * kRowsPerWave + k + (lane >> 4);
                if constexpr (QJL) {  // K half: 8 copies of the fp16 +-1 octet of sign byte e
                    uint4 v4;
                    if (lane & 8) {
                        const uint32_t v = vstage[e];
                        v4 = make_uint4(v, v, v, v);
                    } else {
                        uint32_t wd[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            wd[q] = ((e >> (2 * q)) & 1 ? 0x3C00u : 0xBC00u) |
                                    ((e >> (2 * q + 1)) & 1 ? 0x3C000000u : 0xBC000000u);
                        v4 = make_uint4(wd[0], wd[1], wd[2], wd[3]);
                    }
                    *reinterpret_cast<uint4*>(kv_row(e) + 4 * (lane & 15)) = v4;
                } else {
                    const uint32_t v = stv[k / 4];
                    *reinterpret_cast<uint4*>(kv_row(e) + 4 * (lane & 15)) = make_uint4(v, v, v, v);
                }
            }
        }
        // B operand of QK, built once per workgroup: column i = row i/2, hi (i
        // even) or lo (i odd) part; k-index 8*gq + e of step s is d = 32*gq + 8*s + e.
        for (int ps = w; ps < 4 * NP; ps += kWaves) {
            const int p = ps >> 2, s = ps & 3;
            half8 b;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                b[e] = hi_lo(qs_at(p * kRows + (i >> 1), 32 * gq + 8 * s + e), lo_col);
            bqs[p][s][lane] = __builtin_bit_cast(uint4, b);
        }
        }  // !STAB
        lds_barrier();
        // NP = 1: the B operands in registers; NP >= 2 reads them from LDS per
        // k-step (64 registers fewer in the two-tile loop).
        half8 bq[1][4];
        if constexpr (NP == 1) {
#pragma unroll
            for (int s = 0; s < 4; ++s) bq[0][s] = __builtin_bit_cast(half8, bqs[0][s][lane]);
        }
        // Byte address of this lane's copy of entry 0 of each table; a lookup
        // puts the code byte into byte 1 (entry stride 256 B) with one v_perm.
        const uint32_t lutk = (uint32_t)reinterpret_cast<uintptr_t>((lds_u32*)(kv_row(0) + (lane & 31)));
        const uint32_t lutv = lutk + 128u;
        const uint32_t lut_hi = lutk & 0xFF00u;  // byte 1 of the base, re-added after the perm
        auto lookup = [&](uint32_t word, int b, int table) -> uint32_t {
            const uint32_t base = table ? lutv : lutk;
            const uint32_t a =
                __builtin_amdgcn_perm(word, base, 0x03020000u | ((4u + b) << 8)) + lut_hi;
            return *reinterpret_cast<const lds_u32*>(a);
        };
        // STAB: the S-row address of byte b of word (this lane's copy; its K pair
        // at + kOffKV), and that of a V code byte (S row + 128: its V pair at
        // + kOffKV).
        const uint32_t luts = (uint32_t)reinterpret_cast<uintptr_t>((lds_u32*)&lut[lane & 31]);
        const uint32_t luts_hi = luts & 0xFF00u;
        auto s_addr = [&](uint32_t word, int b, uint32_t off) -> uint32_t {
            return __builtin_amdgcn_perm(word, luts + off, 0x03020000u | ((4u + b) << 8)) + luts_hi;
        };
        auto lds_at = [](uint32_t a, int off) -> uint32_t {
            return *reinterpret_cast<const lds_u32*>(a + off);
        };
        // QJL: the fp16 +-1 octet of sign byte b of word (copy lane % 8).
        const uint32_t lutq =
            (uint32_t)reinterpret_cast<uintptr_t>((lds_u32*)(kv_row(0) + 4 * (lane & 7)));
        auto signs = [&](uint32_t word, int b) -> half8 {
            const uint32_t a =
                __builtin_amdgcn_perm(word, lutq, 0x03020000u | ((4u + b) << 8)) + (lutq & 0xFF00u);
            typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
            return __builtin_bit_cast(half8, *reinterpret_cast<const lds_u32x4*>(a));
        };

        float m_run[NP], l_run[NP];
        f32x4 acc[NP][8];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            m_run[p] = kInitMax;
            l_run[p] = 0.0f;
#pragma unroll
            for (int v = 0; v < 8; ++v) acc[p][v] = (f32x4){0.f, 0.f, 0.f, 0.f};
        }
        bool first = true;
        int slot_nx = load_slot(t0 + kWaves * kChunk);

        // The chunk loop of the one-group layout (NP = 1).
        auto chunk_loop = [&](auto npa) {
            constexpr int NPA = decltype(npa)::value;
            while (t0 < t_end) {  // wave-uniform
                const uint4* kw = cur.kw;
                const uint32_t(*vw)[8] = cur.vw;
                {
                    const float ks = h2f(cur.ks), vs = h2f(cur.vs), re = PROD ? h2f(cur.re) : 0.0f;
                    const float4 sc = QJL    ? make_float4(0.0f, ks * kLog2e, vs, 0.0f)
                                      : PROD ? make_float4(ks * ck, ks * re * cr, vs, 0.0f)
                                             : make_float4(ks * ck, ks * ck * kLoScale, vs, 0.0f);
                    tsc[w][lane & (kChunk - 1)] =
                        cur.valid ? sc : make_float4(0.f, 0.f, 0.f, -INFINITY);
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                Chunk nxt;
                const int t1 = t0 + kWaves * kChunk;
                if (t1 < t_end) {  // codes of the next chunk, slots of the one after
                    fetch(t1, slot_nx, nxt);
                    slot_nx = load_slot(t1 + kWaves * kChunk);
                }

                // The scale rows of this lane's tokens, read before any lookup
                // (LDS reads complete in order: a read issued after the V
                // lookups would wait for all of them).
                float4 scv[kTiles][4];
#pragma unroll
                for (int tau = 0; tau < kTiles; ++tau)
#pragma unroll
                    for (int e = 0; e < 4; ++e) scv[tau][e] = tsc[w][16 * tau + 4 * gq + e];
                // QK: every table lookup of the chunk's K codes is issued before
                // the first MFMA, so their LDS latencies overlap.  prod: aK*K3
                // (table 0); mse: aV*V4 hi parts (table 1) and lo parts (table 0)
                // in kl; QJL: the sign octets.
                half8 ka[kTiles][4], kl[kTiles][4];
#pragma unroll
                for (int tau = 0; tau < kTiles; ++tau) {
                    const uint32_t wd[4] = {kw[tau].x, kw[tau].y, kw[tau].z, kw[tau].w};
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        if constexpr (QJL) {  // sign byte s of the lane's word
                            ka[tau][s] = signs(wd[0], s);
                        } else {
                            const int kt = PROD ? 0 : 1;
                            ka[tau][s] = as_h8(lookup(wd[s], 0, kt), lookup(wd[s], 1, kt),
                                               lookup(wd[s], 2, kt), lookup(wd[s], 3, kt));
                            if constexpr (!PROD)
                                kl[tau][s] = as_h8(lookup(wd[s], 0, 0), lookup(wd[s], 1, 0),
                                                   lookup(wd[s], 2, 0), lookup(wd[s], 3, 0));
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                f32x4 cb[NPA][kTiles], cs[NPA][kTiles];
#pragma unroll
                for (int tau = 0; tau < kTiles; ++tau) {
#pragma unroll
                    for (int p = 0; p < NPA; ++p) {
                        cb[p][tau] = (f32x4){0.f, 0.f, 0.f, 0.f};
                        cs[p][tau] = cb[p][tau];
                    }
                    const uint32_t wd[4] = {kw[tau].x, kw[tau].y, kw[tau].z, kw[tau].w};
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        if constexpr (QJL) {
#pragma unroll
                            for (int p = 0; p < NPA; ++p)
                                cs[p][tau] = mma(ka[tau][s], bq[p][s], cs[p][tau]);
                            continue;
                        }
#pragma unroll
                        for (int p = 0; p < NPA; ++p)
                            cb[p][tau] = mma(ka[tau][s], bq[p][s], cb[p][tau]);
                        if constexpr (!PROD) {  // mse: the lo parts into cs
#pragma unroll
                            for (int p = 0; p < NPA; ++p)
                                cs[p][tau] = mma(kl[tau][s], bq[p][s], cs[p][tau]);
                        } else {
                            // Residual signs (nibble bit 3: 1 -> +1) as fp16 pairs in
                            // registers: high bytes 0x3C / 0xBC, low bytes 0.
                            // even d, odd d
                            const uint32_t he = ((wd[s] << 4) & 0x80808080u) ^ 0xBCBCBCBCu;
                            const uint32_t ho = (wd[s] & 0x80808080u) ^ 0xBCBCBCBCu;
                            const half8 sa = as_h8(__builtin_amdgcn_perm(ho, he, 0x040C000Cu),
                                                   __builtin_amdgcn_perm(ho, he, 0x050C010Cu),
                                                   __builtin_amdgcn_perm(ho, he, 0x060C020Cu),
                                                   __builtin_amdgcn_perm(ho, he, 0x070C030Cu));
#pragma unroll
                            for (int p = 0; p < NPA; ++p)
                                cs[p][tau] = mma(sa, bq[p][s], cs[p][tau]);
                        }
                    }
                }
                // The V lookups (B operands of PV) go out now: the softmax below
                // runs while they are in flight.
                uint32_t bv[kSteps][8][4];  // [step][N-tile v = d - 8i][token pair]
#pragma unroll
                for (int st = 0; st < kSteps; ++st)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t we = vw[st][2 * q], wo = vw[st][2 * q + 1];
                        const uint32_t lob = (we & 0x0F0F0F0Fu) | ((wo & 0x0F0F0F0Fu) << 4);
                        const uint32_t hib = ((we >> 4) & 0x0F0F0F0Fu) | (wo & 0xF0F0F0F0u);
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            bv[st][2 * b][q] = lookup(lob, b, 1);
                            bv[st][2 * b + 1][q] = lookup(hib, b, 1);
                        }
                    }
                __builtin_amdgcn_sched_barrier(0);
                // Logits (base 2) of tokens 16*tau + 4*gq + e; hi + lo columns summed.
                float lg[NPA][kTiles][4];
#pragma unroll
                for (int p = 0; p < NPA; ++p) {
                    // rows shorter than the chunk's end need the causal mask
                    const bool masked = PAGED && t0 + kChunk > gmin[p];
                    float mloc = -INFINITY;
#pragma unroll
                    for (int tau = 0; tau < kTiles; ++tau)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float4 sc = scv[tau][e];
                            if constexpr (QJL) {
                                const float sr = cs[p][tau][e] + quad_xor<1>(cs[p][tau][e]);
                                lg[p][tau][e] = fmaf(sr, sc.y, sc.w);
                            } else {
                                const float sb = cb[p][tau][e] + quad_xor<1>(cb[p][tau][e]);
                                const float sr = cs[p][tau][e] + quad_xor<1>(cs[p][tau][e]);
                                lg[p][tau][e] = fmaf(sb, sc.x, fmaf(sr, sc.y, sc.w));
                            }
                            if (masked)  // causal limit of this column's row
                                if (t0 + 16 * tau + 4 * gq + e >= rowlen[p])
                                    lg[p][tau][e] = -INFINITY;
                            mloc = fmaxf(mloc, lg[p][tau][e]);
                        }
                    mloc = lane_xor_reduce<16>(mloc, [](float x, float y) { return fmaxf(x, y); });
                    mloc = lane_xor_reduce<32>(mloc, [](float x, float y) { return fmaxf(x, y); });
                    // v_exp_f32 without denormal handling: arguments are <= 0 and a
                    // weight below 2^-126 of the running maximum is negligible.
                    const float m_new = fmaxf(m_run[p], mloc);
                    const float alpha = first ? 0.0f : __builtin_amdgcn_exp2f(m_run[p] - m_new);
                    m_run[p] = m_new;
                    float lsum = 0.0f;
#pragma unroll
                    for (int tau = 0; tau < kTiles; ++tau)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            lg[p][tau][e] = __builtin_amdgcn_exp2f(lg[p][tau][e] - m_new);
                            lsum += lg[p][tau][e];
                        }
                    l_run[p] = l_run[p] * alpha + lsum;
                    if (!first && __any(alpha != 1.0f)) {
                        // acc lane (d, gq) holds columns 4gq..4gq+3 = rows 2gq, 2gq+1.
                        const float a0 = __shfl(alpha, 4 * gq), a1 = __shfl(alpha, 4 * gq + 2);
#pragma unroll
                        for (int v = 0; v < 8; ++v) {
                            acc[p][v][0] *= a0;
                            acc[p][v][1] *= a0;
                            acc[p][v][2] *= a1;
                            acc[p][v][3] *= a1;
                        }
                    }
                }
                // PV: one decoded B operand per N-tile, an MFMA per position
#pragma unroll
                for (int st = 0; st < kSteps; ++st) {
                    half8 ap[NPA];
#pragma unroll
                    for (int p = 0; p < NPA; ++p)
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const int tau = 2 * st + (e >> 2), ee = e & 3;
                            ap[p][e] = hi_lo(lg[p][tau][ee] * scv[tau][ee].z, lo_col);
                        }
#pragma unroll
                    for (int v = 0; v < 8; ++v) {
                        const half8 bvv =
                            as_h8(bv[st][v][0], bv[st][v][1], bv[st][v][2], bv[st][v][3]);
#pragma unroll
                        for (int p = 0; p < NPA; ++p)
                            acc[p][v] = mma(ap[p], bvv, acc[p][v]);
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                cur = nxt;
                t0 = t1;
                first = false;
            }
        };
        // NP >= 2: one softmax state per lane and tile (its column's row), hi and
        // lo stacked along the reductions.  A unit with fewer positions runs the
        // loop over the tiles it needs; a tile's unused columns compute on zero
        // queries and are dropped.
        float m_col[NT], l_col[NT];
        f32x4 acc_col[NT][8];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            m_col[t] = kInitMax;
            l_col[t] = 0.0f;
#pragma unroll
            for (int v = 0; v < 8; ++v) acc_col[t][v] = (f32x4){0.f, 0.f, 0.f, 0.f};
        }
        // COLS (a unit of one position): one tile whose columns are the
        // position's rows as hi (columns 0-7) and lo (8-15) parts, as in the
        // one-group kernel: one MFMA per product instead of two, and the two
        // halves of a column pair summed (logits; outputs at the merge).
        auto stacked_loop = [&](auto nta, auto cols) {
            constexpr int NTA = decltype(nta)::value;
            constexpr bool COLS = decltype(cols)::value;
            static_assert(!COLS || NTA == 1, "one tile");
            while (t0 < t_end) {  // wave-uniform
                const uint4* kw = cur.kw;
                const uint32_t(*vw)[8] = cur.vw;
                {
                    const float ks = h2f(cur.ks), vs = h2f(cur.vs), re = PROD ? h2f(cur.re) : 0.0f;
                    tsc[w][lane & (kChunk - 1)] =
                        cur.valid ? make_float4(ks * ck, PROD ? ks * re * cr : ks * ck * kLoScale,
                                                0.5f * vs, 0.0f)
                                  : make_float4(0.f, 0.f, 0.f, -INFINITY);
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const int t1 = t0 + kWaves * kChunk;
                // QK: each decoded A operand against every tile's hi and lo query
                f32x4 cb[NTA][kTiles], cs[NTA][kTiles];
#pragma unroll
                for (int tau = 0; tau < kTiles; ++tau)
#pragma unroll
                    for (int t = 0; t < NTA; ++t) {
                        cb[t][tau] = (f32x4){0.f, 0.f, 0.f, 0.f};
                        cs[t][tau] = cb[t][tau];
                    }
                // The operands of k-step s + 1 (query parts, decoded codes) are
                // read from LDS before the MFMAs of step s.
                struct Ops {
                    half8 bk[2 * NTA];  // k-step s of each tile's hi and lo query
                    half8 a[kTiles], al[kTiles];
                };
                auto load_ops = [&](int s, Ops& o) {
#pragma unroll
                    for (int pp = 0; pp < (COLS ? 1 : 2 * NTA); ++pp)
                        o.bk[pp] = __builtin_bit_cast(half8, bqs[pp][s][lane]);
#pragma unroll
                    for (int tau = 0; tau < kTiles; ++tau) {
                        const uint32_t wd = s == 0   ? kw[tau].x
                                            : s == 1 ? kw[tau].y
                                            : s == 2 ? kw[tau].z
                                                     : kw[tau].w;
                        // one address per byte: its K pair (prod aK*K3, mse the hi
                        // parts) and its S pair (prod the residual signs, mse the lo
                        // parts)
                        uint32_t ad[4];
#pragma unroll
                        for (int b = 0; b < 4; ++b) ad[b] = s_addr(wd, b, 0);
                        o.a[tau] = as_h8(lds_at(ad[0], kOffKV), lds_at(ad[1], kOffKV),
                                         lds_at(ad[2], kOffKV), lds_at(ad[3], kOffKV));
                        o.al[tau] = as_h8(lds_at(ad[0], 0), lds_at(ad[1], 0), lds_at(ad[2], 0),
                                          lds_at(ad[3], 0));
                    }
                };
                Ops ops[2];
                float4 scq[kTiles][4];  // the logits' per-token scales, read during the last k-step
                load_ops(0, ops[0]);
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    if (s < 3) {
                        load_ops(s + 1, ops[(s + 1) & 1]);
                    } else {
#pragma unroll
                        for (int tau = 0; tau < kTiles; ++tau)
#pragma unroll
                            for (int e = 0; e < 4; ++e) scq[tau][e] = tsc[w][16 * tau + 4 * gq + e];
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    const Ops& o = ops[s & 1];
#pragma unroll
                    for (int tau = 0; tau < kTiles; ++tau) {
#pragma unroll
                        for (int t = 0; t < NTA; ++t) {
                            cb[t][tau] = mma(o.a[tau], o.bk[2 * t], cb[t][tau]);
                            if (!COLS) cb[t][tau] = mma(o.a[tau], o.bk[2 * t + 1], cb[t][tau]);
                        }
                        // prod: the +-1 residual signs against the hi and lo query;
                        // mse: the codebook's lo parts (into cs) against the hi query
                        // only: the product of the two lo parts, each below 2^-11
                        // of its value, is ~2^-22 of the logit
#pragma unroll
                        for (int t = 0; t < NTA; ++t) {
                            cs[t][tau] = mma(o.al[tau], o.bk[2 * t], cs[t][tau]);
                            if (!COLS && PROD)
                                cs[t][tau] = mma(o.al[tau], o.bk[2 * t + 1], cs[t][tau]);
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                const bool masked = t0 + kChunk > gmin_live;
                // Logits (base 2) of tokens 16*tau + 4*gq + e for this lane's column.
                float lg[NTA][kTiles][4];
#pragma unroll
                for (int t = 0; t < NTA; ++t)
#pragma unroll
                    for (int tau = 0; tau < kTiles; ++tau)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float4 sc = scq[tau][e];
                            float b = cb[t][tau][e], r = cs[t][tau][e];
                            if constexpr (COLS) {  // + the partner column (lane ^ 8)
                                b += lane_xor<8>(b);
                                r += lane_xor<8>(r);
                            }
                            lg[t][tau][e] = fmaf(b, sc.x, fmaf(r, sc.y, sc.w));
                        }
                // The V lookups (B operands of PV) go out before the softmax,
                // whose VALU work hides their LDS latency.
                uint32_t bv[kSteps][8][4];  // [step][N-tile v = d - 8i][token pair]
#pragma unroll
                for (int st = 0; st < kSteps; ++st)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t we = vw[st][2 * q], wo = vw[st][2 * q + 1];
                        const uint32_t lob = (we & 0x0F0F0F0Fu) | ((wo & 0x0F0F0F0Fu) << 4);
                        const uint32_t hib = ((we >> 4) & 0x0F0F0F0Fu) | (wo & 0xF0F0F0F0u);
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            // (turbo_prod: the V copies; turbo_mse: its K copies hold aV*V4)
                            bv[st][2 * b][q] = lds_at(s_addr(lob, b, PROD ? 128u : 0u), kOffKV);
                            bv[st][2 * b + 1][q] = lds_at(s_addr(hib, b, PROD ? 128u : 0u), kOffKV);
                        }
                    }
                __builtin_amdgcn_sched_barrier(0);
                // This chunk's codes are consumed: the next chunk's codes and the
                // slots of the one after are fetched into cur's registers, in
                // flight during the softmax and PV (no copy at the end of the
                // step, which would wait for them: 128.3 -> 127.1 us turbo_prod,
                // 129.5 -> 127.1 us turbo_mse against fetching into a second
                // buffer behind the first k-step).
                if (t1 < t_end) {
                    fetch(t1, slot_nx, cur);
                    slot_nx = load_slot(t1 + kWaves * kChunk);
                }
                if (masked) {  // a row of the unit ends in this chunk (wave-uniform)
                    asm volatile("" ::: "memory");  // a branch: no selects on every chunk
#pragma unroll
                    for (int t = 0; t < NTA; ++t)
#pragma unroll
                        for (int tau = 0; tau < kTiles; ++tau)
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                if (t0 + 16 * tau + 4 * gq + e >= rl_col[t])
                                    lg[t][tau][e] = -INFINITY;
                }
                // Online softmax with a lagging maximum: m_col moves (and the
                // accumulators are rescaled) only when a logit passes it by more
                // than 1, so the weights stay <= 2 (the PV operand is P * vs / 2).
                float mloc[NTA];
                bool grow = false;
#pragma unroll
                for (int t = 0; t < NTA; ++t) {
                    // (IEEE maximum: no canonicalising of the lane-exchanged
                    // values; a NaN logit leaves grow false, as fmaxf would)
                    float m = lg[t][0][0];
#pragma unroll
                    for (int k = 1; k < 4 * kTiles; ++k)
                        m = __builtin_elementwise_maximum(m, lg[t][k >> 2][k & 3]);
                    const auto mx = [](float x, float y) { return __builtin_elementwise_maximum(x, y); };
                    m = lane_xor_reduce<16>(m, mx);
                    mloc[t] = lane_xor_reduce<32>(m, mx);
                    grow = grow || mloc[t] > m_col[t] + 1.0f;
                }
                if (__any(grow)) {  // wave-uniform
#pragma unroll
                    for (int t = 0; t < NTA; ++t) {
                        const float m_new = fmaxf(m_col[t], mloc[t]);
                        const float alpha = __builtin_amdgcn_exp2f(m_col[t] - m_new);
                        m_col[t] = m_new;
                        l_col[t] *= alpha;
                        // acc lane (d, gq) holds rows 4gq .. 4gq + 3 (columns of lanes 4gq + e)
                        float a[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) a[e] = __shfl(alpha, 4 * gq + e);
#pragma unroll
                        for (int v = 0; v < 8; ++v)
#pragma unroll
                            for (int e = 0; e < 4; ++e) acc_col[t][v][e] *= a[e];
                    }
                }
#pragma unroll
                for (int t = 0; t < NTA; ++t) {
#pragma unroll
                    for (int tau = 0; tau < kTiles; ++tau)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            lg[t][tau][e] = __builtin_amdgcn_exp2f(lg[t][tau][e] - m_col[t]);
                    // pairwise: no zero start, and the adds do not wait on one another
                    float part[kTiles];
#pragma unroll
                    for (int tau = 0; tau < kTiles; ++tau)
                        part[tau] = (lg[t][tau][0] + lg[t][tau][1]) + (lg[t][tau][2] + lg[t][tau][3]);
                    float lsum = part[0];
#pragma unroll
                    for (int tau = 1; tau < kTiles; ++tau) lsum += part[tau];
                    l_col[t] += lsum;
                }
                // PV: every tile's hi and lo P against each decoded B operand
#pragma unroll
                for (int st = 0; st < kSteps; ++st) {
                    half8 ah[NTA], al[NTA];
#pragma unroll
                    for (int t = 0; t < NTA; ++t) {
                        uint32_t hw[4], lw[4];
#pragma unroll
                        for (int e = 0; e < 8; e += 2) {
                            const int tau = 2 * st + (e >> 2), ee = e & 3;
                            const float x0 = lg[t][tau][ee] * tsc[w][16 * tau + 4 * gq + ee].z;
                            const float x1 =
                                lg[t][tau][ee + 1] * tsc[w][16 * tau + 4 * gq + ee + 1].z;
                            hw[e >> 1] = pack_h2(x0, x1);
                            lw[e >> 1] = lo_pair(x0, x1, hw[e >> 1]);
                        }
                        if constexpr (COLS) {  // column i < 8: hi; i >= 8: lo
                            const bool lo = (i >> 3) != 0;
                            ah[t] = as_h8(lo ? lw[0] : hw[0], lo ? lw[1] : hw[1], lo ? lw[2] : hw[2],
                                          lo ? lw[3] : hw[3]);
                        } else {
                            ah[t] = as_h8(hw[0], hw[1], hw[2], hw[3]);
                            al[t] = as_h8(lw[0], lw[1], lw[2], lw[3]);
                        }
                    }
#pragma unroll
                    for (int v = 0; v < 8; ++v) {
                        const half8 bvv =
                            as_h8(bv[st][v][0], bv[st][v][1], bv[st][v][2], bv[st][v][3]);
#pragma unroll
                        for (int t = 0; t < NTA; ++t) {
                            acc_col[t][v] = mma(ah[t], bvv, acc_col[t][v]);
                            if (!COLS) acc_col[t][v] = mma(al[t], bvv, acc_col[t][v]);
                        }
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                t0 = t1;
                first = false;
            }
        };
        if constexpr (NP >= 2) {
            if (NT == 2 && ntile == 2)
                stacked_loop(std::integral_constant<int, NT>{}, std::false_type{});
            else if (npos == 1)
                stacked_loop(std::integral_constant<int, 1>{}, std::true_type{});
            else
                stacked_loop(std::integral_constant<int, 1>{}, std::false_type{});
        } else {
            chunk_loop(std::integral_constant<int, 1>{});
        }

        // Wave results: l summed over the g lanes of each column; o rows (NP = 1:
        // from the hi + lo columns), the V codebook scale divided out.  Then the
        // waves are merged per row, the inverse WHT and sign flip applied, and the
        // partial written to the workspace (NP >= 2: one tile of 16 rows per pass
        // through the merge space).  A position whose rows all end before this
        // piece has no partial (its combine reads only the pieces below its
        // longest row).
        if constexpr (NP >= 2) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float l_tot = lane_xor_reduce<16>(l_col[t], [](float x, float y) { return x + y; });
                l_tot = lane_xor_reduce<32>(l_tot, [](float x, float y) { return x + y; });
                if (gq == 0) {
                    mm[w][16 * t + i] = m_col[t];
                    ml[w][16 * t + i] = l_tot;
                }
            }
        } else {
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                float l_tot = lane_xor_reduce<16>(l_run[p], [](float x, float y) { return x + y; });
                l_tot = lane_xor_reduce<32>(l_tot, [](float x, float y) { return x + y; });
                if (gq == 0 && !lo_col) {
                    mm[w][p * kRows + (i >> 1)] = m_run[p];
                    ml[w][p * kRows + (i >> 1)] = l_tot;
                }
            }
        }
        const float iav = 1.0f / kAlphaV;
        const float s0 = (!QJL && (h & 1)) ? -inv : inv;
        // Row rr of tile t from the merge space mt (the 8 waves' o rows): the
        // waves' (m, l, o) merged, the inverse WHT and sign flip, the partial.
        auto merge_row = [&](int t, int rr, float(*mt)[kMoRows][128]) {
            const int r = kMoRows * t + rr;  // row of the workgroup
            const int p = r / kRows;
            bool keep = p < npos;
            if constexpr (PAGED) keep = keep && t_begin < gend[p];
            if (!keep) return;  // wave-uniform
            float M = mm[0][r];
#pragma unroll
            for (int u = 1; u < kWaves; ++u) M = fmaxf(M, mm[u][r]);
            float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
            for (int u = 0; u < kWaves; ++u) {
                const float wt = __builtin_amdgcn_exp2f(mm[u][r] - M);  // (argument <= 0)
                L += ml[u][r] * wt;
                o0 += mt[u][rr][2 * lane] * wt;
                o1 += mt[u][rr][2 * lane + 1] * wt;
            }
            if (NP >= 2 && npos == 1) {  // one position: + its lo columns 8-15
#pragma unroll
                for (int u = 0; u < kWaves; ++u) {
                    const float wt = __builtin_amdgcn_exp2f(mm[u][r] - M);  // (argument <= 0)
                    o0 += mt[u][rr + kRows][2 * lane] * wt;
                    o1 += mt[u][rr + kRows][2 * lane + 1] * wt;
                }
            }
            wht_pair<64>(o0, o1, lane);
            float* part = ws + ((pid * NP + p) * kRows + r % kRows) * kPartStride;
            part[2 * lane] = o0 * s0;
            part[2 * lane + 1] = o1 * -s0;
            if (lane == 0) {
                part[128] = M;
                part[129] = L;
            }
        };
        if constexpr (NP >= 2) {
            // Both tiles at once: tile t's merge space at table word 16384 t
            // (the tables are no longer read), three barriers per piece instead
            // of four, and each wave's four rows merged without a barrier
            // between them.
            static_assert(NT * sizeof(float) * kWaves * kMoRows * 128 <= sizeof(lut), "merge spaces");
            auto mot = [&](int t) { return reinterpret_cast<float(*)[kMoRows][128]>(&lut[16384 * t]); };
            __syncthreads();  // every wave is done with the tables
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (t >= ntile) break;  // wave- and workgroup-uniform
#pragma unroll
                for (int v = 0; v < 8; ++v)
#pragma unroll
                    for (int e = 0; e < 4; ++e)  // (x2: the PV operand was P * vs / 2)
                        mot(t)[w][4 * gq + e][8 * i + v] = acc_col[t][v][e] * (2.0f * iav);
            }
            __syncthreads();
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int k = 0; k < kMoRows / kWaves; ++k) merge_row(t, w + k * kWaves, mot(t));
            // the next piece's setup writes its rotated queries into the S rows,
            // which hold tile 0's merge space
            __syncthreads();
        } else {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                __syncthreads();  // every wave is done with the tables (or the last pass) mo overwrites
#pragma unroll
                for (int p = 0; p < NP; ++p)
#pragma unroll
                    for (int v = 0; v < 8; ++v) {
                        mo[w][p * kRows + 2 * gq][8 * i + v] = (acc[p][v][0] + acc[p][v][1]) * iav;
                        mo[w][p * kRows + 2 * gq + 1][8 * i + v] =
                            (acc[p][v][2] + acc[p][v][3]) * iav;
                    }
                __syncthreads();
                for (int rr = w; rr < kMoRows; rr += kWaves) merge_row(t, rr, mo);
            }
        }
    };  // item

    if constexpr (PAGED) {
        // Every kv head has the same work (the units' passes over their kv
        // lengths), split into Gh = G / H segments; workgroup b takes head
        // b / Gh and segment seg(b % Gh) of it.  Gh is a multiple of 8 and
        // workgroup b runs on XCD b % 8, so the H workgroups of one segment
        // share an XCD and walk the same tokens at the same time: the heads
        // of a token share its cache lines (cell tib * H + h), and the second
        // reader finds them in that XCD's L2.  The segments of one XCD are
        // consecutive, so the units of a sequence mostly share it too.
        constexpr int kPass = kChunk * kWaves;
        const int Gh = (int)gridDim.x / g.H;
        const int hh = (int)blockIdx.x / Gh;
        const int bl = (int)blockIdx.x - hh * Gh;
        const int seg = (bl & 7) * (Gh >> 3) + (bl >> 3);
        const int nu = __builtin_amdgcn_readfirstlane(pr.plan[0]);
        const int total = __builtin_amdgcn_readfirstlane(pr.plan[1]);
        const Segments sg(total, Gh);
        const int b0 = sg.bound(seg), b1 = sg.bound(seg + 1);
        if (b0 >= b1) return;  // an empty segment (less work than workgroups)
        // The unit holding work position b0: exactly one u has start(u) <= b0 <
        // start(u + 1), or b0 lies before the first unit's first pass (unit 0).
        __shared__ int s_unit;
        for (int u = threadIdx.x; u < nu; u += 64 * kWaves)
            if ((u == 0 || pr.units[u].start <= b0) && b0 < pr.units[u + 1].start) s_unit = u;
        __syncthreads();
        // The walk over the units overlapping the segment, in work order.  Its
        // position lives in LDS (one copy per wave, volatile accesses), so no
        // walk state is held in registers across an item.  The pointer is an
        // LDS one: a generic (flat) access would also wait for the previous
        // piece's partial stores.
        __shared__ int s_walk[kWaves];
        typedef __attribute__((address_space(3))) int lds_int;
        const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        volatile lds_int* walk = (volatile lds_int*)&s_walk[wv];
        if ((threadIdx.x & 63) == 0) walk[0] = __builtin_amdgcn_readfirstlane(s_unit);
        for (;;) {
            const int u = __builtin_amdgcn_readfirstlane(walk[0]);
            if (u >= nu) break;
            const PagedUnit un = pr.units[u];
            if (un.start >= b1) break;
            if ((threadIdx.x & 63) == 0) walk[0] = u + 1;
            int x0, x1;
            item_passes(un.start, un.n, un.w, b0, b1, x0, x1);
            if (x0 < x1) {
                int tid = threadIdx.x;
                asm volatile("" : "+v"(tid));  // opaque per item (see item)
                // partial slot: (unit + segment) * H + head, unique (the
                // pieces of one head form a staircase in (unit, segment))
                item(tid, hh, un.first, un.npos, x0 * kPass, min(x1 * kPass, un.kv_end),
                     (size_t)(u + seg) * g.H + hh);
            }
        }
    } else {
        // Grid (split, kv head, row group), or one dimension of splits x heads
        // when there are more row groups than a grid dimension holds (the
        // first form needs no divisions before the first loads).
        int split, h, rg;
        if (gridDim.x == (unsigned)num_splits) {
            split = blockIdx.x;
            h = blockIdx.y;
            rg = blockIdx.z;
        } else {
            split = blockIdx.x % num_splits;
            const int hr = blockIdx.x / num_splits;
            h = hr % g.H;
            rg = hr / g.H;
        }
        const int t_begin = split * tokens_per_split;
        item(threadIdx.x, h, rg, 1, t_begin, t_begin + tokens_per_split,
             ((size_t)rg * g.H + h) * num_splits + split);
    }
}
// Sum of the split partials of one output row (q, h): o = sum_s 2^(m_s - M)
// o_s / sum_s 2^(m_s - M) l_s.  Block = (row, 32-element slice of d), 256
// threads = 8 groups x 32 d.  Group g takes splits g, g + 8, ...: it loads up
// to 16 partials' (m, l, o[d]) in one round, merges them with a running
// maximum, and the 8 groups are merged in LDS.
__global__ __launch_bounds__(256) void attn_mfma_combine_kernel(const float* __restrict__ ws,
                                                                uint16_t* __restrict__ output,
                                                                int H, int num_splits) {
    using namespace mfma;
    constexpr int kBatch = 16;
    __shared__ float red_m[8], red_l[8];
    __shared__ float red_o[8][33];
    // Grid (slice, kv head, query), or one dimension of 4 x rows when there
    // are more queries than a grid dimension holds; row = q * H + h.
    int dq, h, q;
    if (gridDim.x == 4) {
        dq = blockIdx.x;
        h = blockIdx.y;
        q = blockIdx.z;
    } else {
        dq = blockIdx.x & 3;
        const int rw = blockIdx.x >> 2;
        q = rw / H;
        h = rw - q * H;
    }
    const int row = q * H + h;
    const int rg = q / kRows, r = q % kRows;
    const int t = threadIdx.x, dd = t & 31, sg = t >> 5;
    const int d = 32 * dq + dd;
    const size_t base_bid = (size_t)(rg * H + h) * num_splits;
    auto part = [&](int s) { return ws + ((base_bid + s) * kRows + r) * kPartStride; };
    const int S = num_splits;

    float M = kInitMax, L = 0.f, acc = 0.f;
    for (int base = sg; base < S; base += 8 * kBatch) {
        float pm[kBatch], pl[kBatch], po[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int s = base + 8 * k;
            const float* p = part(s < S ? s : base);
            const float2 ml2 = *reinterpret_cast<const float2*>(p + 128);  // (m, l)
            pm[k] = s < S ? ml2.x : kInitMax;
            pl[k] = ml2.y;
            po[k] = p[d];
        }
        float mb = M;
#pragma unroll
        for (int k = 0; k < kBatch; ++k) mb = fmaxf(mb, pm[k]);
        // v_exp_f32 without denormal handling: arguments are <= 0 and a weight
        // below 2^-126 of the largest is negligible.
        const float sc = __builtin_amdgcn_exp2f(M - mb);
        L *= sc;
        acc *= sc;
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const float wt = __builtin_amdgcn_exp2f(pm[k] - mb);
            L += pl[k] * wt;
            acc += po[k] * wt;
        }
        M = mb;
    }
    if (dd == 0) {
        red_m[sg] = M;
        red_l[sg] = L;
    }
    red_o[sg][dd] = acc;
    __syncthreads();
    if (t < 32) {
        float Mx = red_m[0];
#pragma unroll
        for (int u = 1; u < 8; ++u) Mx = fmaxf(Mx, red_m[u]);
        float Lt = 0.f, o = 0.f;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float wt = __builtin_amdgcn_exp2f(red_m[u] - Mx);
            Lt += red_l[u] * wt;
            o += red_o[u][t] * wt;
        }
        output[(size_t)row * 128 + 32 * dq + t] = f2h(Lt > 0.f ? o / Lt : o);
    }
}

// The same merge for few splits: one block per (row group, kv head) item,
// thread t takes row t / 32 and elements 4(t % 32) .. +3 over every split
// (8 in flight).  One block per item instead of 4 per row: for the many short
// items of a batched decode step the block count, not the bytes, is the cost.
constexpr int kItemCombineMaxSplits = 32;
__global__ __launch_bounds__(256) void attn_mfma_combine_items_kernel(
    const float* __restrict__ ws, uint16_t* __restrict__ output, int H, int num_splits,
    int num_queries) {
    using namespace mfma;
    const int item = blockIdx.x;  // h + H * rg
    const int h = item % H, rg = item / H;
    const int t = threadIdx.x, r = t >> 5, d0 = 4 * (t & 31);
    const int S = num_splits;
    const float* base = ws + ((size_t)item * num_splits * kRows + r) * kPartStride;
    float M = kInitMax, L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int b = 0; b < S; b += 8) {
        float pm[8], pl[8];
        float4 po[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const bool ok = b + k < S;
            const float* p = base + (size_t)min(b + k, S - 1) * kRows * kPartStride;
            pm[k] = ok ? p[128] : kInitMax;
            pl[k] = ok ? p[129] : 0.f;
            po[k] = ok ? *reinterpret_cast<const float4*>(p + d0) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float mb = M;
#pragma unroll
        for (int k = 0; k < 8; ++k) mb = fmaxf(mb, pm[k]);
        const float sc = __builtin_amdgcn_exp2f(M - mb);  // (argument <= 0)
        L *= sc;
        acc.x *= sc;
        acc.y *= sc;
        acc.z *= sc;
        acc.w *= sc;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float wt = __builtin_amdgcn_exp2f(pm[k] - mb);
            L += pl[k] * wt;
            acc.x += po[k].x * wt;
            acc.y += po[k].y * wt;
            acc.z += po[k].z * wt;
            acc.w += po[k].w * wt;
        }
        M = mb;
    }
    const int q = rg * kRows + r;
    if (q >= num_queries) return;
    const auto fin = [&](float o) { return (uint32_t)f2h(L > 0.f ? o / L : o); };
    *reinterpret_cast<uint2*>(output + ((size_t)q * H + h) * 128 + d0) =
        make_uint2(fin(acc.x) | (fin(acc.y) << 16), fin(acc.z) | (fin(acc.w) << 16));
}

// Merge of a paged step's partials: one block per (row group, kv head), laid
// out as in attn_mfma_combine_items_kernel.  The row group is position p of
// unit u; its item's passes were cut at segment bounds into pieces, one
// partial per segment they start in (slot item + segment, position p), and
// a piece starting at or past the group's longest row wrote none.
__global__ __launch_bounds__(256) void attn_paged_combine_kernel(
    const float* __restrict__ ws, uint16_t* __restrict__ output, int H, int num_queries,
    int num_segments, int positions, int pass, mfma::PagedRows pr) {
    using namespace mfma;
    const int item = blockIdx.x;  // h + H * rg
    const int h = item % H, rg = item / H;
    const int t = threadIdx.x, r = t >> 5, d0 = 4 * (t & 31);
    const PagedUnit un = pr.group_unit[rg];
    const int u = un.index;
    const int total = pr.plan[1], G = num_segments;
    const int p = rg - un.first;
    // The group's longest row: the row lengths are loaded unconditionally (a
    // row past the end re-reads the last row), so the loads go out together
    // with the unit's record instead of one after another in branches.
    int kvr[kRows];
#pragma unroll
    for (int k = 0; k < kRows; ++k) kvr[k] = pr.row_kv_len[min(rg * kRows + k, num_queries - 1)];
    int kv = 0;
#pragma unroll
    for (int k = 0; k < kRows; ++k)
        if (rg * kRows + k < num_queries) kv = max(kv, kvr[k]);
    const int S = un.start;  // every head has the unit's work range, in its own segments
    // segments holding the item's first and last pass starts
    int g_lo = 0, g_hi = -1;
    const Segments sg(max(total, 1), G);
    if (un.n > 0 && kv > 0) {
        g_lo = sg.of(S, total);
        g_hi = sg.of(S + un.w * (un.n - 1), total);
    }
    const size_t unit0 = (size_t)u;
    float M = kInitMax, L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int b = g_lo; b <= g_hi; b += 8) {
        float pm[8], pl[8];
        float4 po[8];
        float2 mlr[8];
        int okv[8];
        // (slot gs <= g_hi is one of the item's pieces: the loads are
        // unconditional and all in flight together; the pieces that wrote
        // nothing are dropped after, by a per-lane select rather than a branch
        // whose join would wait for each load in turn)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int gs = min(b + k, g_hi);
            int x0, x1;
            item_passes(S, un.n, un.w, sg.bound(gs), sg.bound(gs + 1), x0, x1);
            okv[k] = b + k <= g_hi && x0 < x1 && x0 * pass < kv;
            const float* pp =
                ws + ((((unit0 + gs) * H + h) * positions + p) * kRows + r) * kPartStride;
            mlr[k] = *reinterpret_cast<const float2*>(pp + 128);
            po[k] = *reinterpret_cast<const float4*>(pp + d0);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            int ok = okv[k];
            asm volatile("" : "+v"(ok));
            pm[k] = ok ? mlr[k].x : kInitMax;
            pl[k] = ok ? mlr[k].y : 0.f;
            if (!ok) po[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float mb = M;
#pragma unroll
        for (int k = 0; k < 8; ++k) mb = fmaxf(mb, pm[k]);
        const float sc = __builtin_amdgcn_exp2f(M - mb);  // (argument <= 0)
        L *= sc;
        acc.x *= sc;
        acc.y *= sc;
        acc.z *= sc;
        acc.w *= sc;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float wt = __builtin_amdgcn_exp2f(pm[k] - mb);
            L += pl[k] * wt;
            acc.x += po[k].x * wt;
            acc.y += po[k].y * wt;
            acc.z += po[k].z * wt;
            acc.w += po[k].w * wt;
        }
        M = mb;
    }
    const int q = rg * kRows + r;
    if (q >= num_queries) return;
    const auto fin = [&](float o) { return (uint32_t)f2h(L > 0.f ? o / L : o); };
    *reinterpret_cast<uint2*>(output + ((size_t)q * H + h) * 128 + d0) =
        make_uint2(fin(acc.x) | (fin(acc.y) << 16), fin(acc.z) | (fin(acc.w) << 16));
}

// Inclusive scan over the 1024 threads of a block (16 waves) with an
// associative op: within each wave by shuffles, then over the wave totals.
template <typename Op>
__device__ int block_scan_1024(int v, int ident, int* s_tot, Op op) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(v, d);
        if (lane >= d) v = op(v, o);
    }
    if (lane == 63) s_tot[wv] = v;
    __syncthreads();
    // The earlier waves' totals: all 16 read at once (one LDS round trip),
    // then combined below this wave's index.
    int tot[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) tot[k] = s_tot[k];
    int pre = ident;
#pragma unroll
    for (int k = 0; k < 16; ++k)
        if (k < wv) pre = op(pre, tot[k]);
    __syncthreads();  // s_tot is reused by the next scan
    return op(pre, v);
}

// Paged steps: the work positions a unit's setup counts for (a two-tile pass
// weighs 4), before its first pass (config 5, 32 sequences: 139 us per step
// with 0, 135 with 4, 131-133 with 8, 12 or 16).
#ifndef TQ_PAGED_PIECE_COST
#define TQ_PAGED_PIECE_COST 8
#endif
constexpr int kPieceCost = TQ_PAGED_PIECE_COST;

// The plan of a paged step, one block of 1024 threads.  Row groups (8 rows
// of one sequence) form units: each run of consecutive groups of one
// sequence is cut into units of U groups from its start, the last one
// shorter.  A unit's items (one per kv head) are n = ceil(kv_end / pass)
// passes over its longest row (at most max_kv_len), a pass weighing w: with
// U = 4, 4 for a unit of more than two positions (the two-tile loop) and 3
// otherwise, about their measured cost ratio.  Work positions are given out
// in unit order; a unit with passes first takes kPieceCost positions that no
// pass occupies (its start is its first pass): a workgroup pays a piece's
// setup (query rotation, decode tables, a first chunk with nothing in flight)
// for every unit it starts, so a segment holding unit starts gets less pass
// work.  The groups are taken 1024 at a time, carrying the run start, the
// unit count and the work total from window to window.
template <int U>
__global__ __launch_bounds__(1024) void paged_plan_kernel(
    const int32_t* __restrict__ row_seq, const int32_t* __restrict__ row_kv_len, int num_rows,
    int groups, int pass, int max_kv_len, mfma::PagedUnit* __restrict__ units,
    mfma::PagedUnit* __restrict__ group_unit, int32_t* __restrict__ plan) {
    static_assert(U >= 1 && U <= 4 && (U & (U - 1)) == 0, "1, 2 or 4 groups per unit");
    using mfma::kRows;
    constexpr int kWin = 1024;
    __shared__ int s_sq[kWin + U], s_gk[kWin + U], s_tot[16], s_carry[4];
    const int j = threadIdx.x;
    // The group's longest row (rows past num_rows: 0).  The loads are
    // unconditional (a row past the end re-reads the last row), so the eight
    // go out together: a load under a condition sits in a branch whose join
    // waits for it, one memory latency per row.
    auto load_kv = [&](int gi, int (&v)[kRows]) {
#pragma unroll
        for (int k = 0; k < kRows; ++k) v[k] = row_kv_len[min(gi * kRows + k, num_rows - 1)];
    };
    auto group_kv = [&](int gi, const int (&v)[kRows]) {
        int m = 0;
#pragma unroll
        for (int k = 0; k < kRows; ++k)
            if (gi * kRows + k < num_rows) m = max(m, v[k]);
        return min(m, max_kv_len);
    };
    const auto add = [](int a, int b) { return a + b; };
    const auto mx = [](int a, int b) { return max(a, b); };
    int c_units = 0, c_work = 0, c_rs = 0, c_sq = 0;
    for (int base = 0; base < groups; base += kWin) {
        const int gi = base + j;
        const bool in = gi < groups;
        // (groups past the end load the last group, unconditionally, then drop it)
        const int gc = min(gi, groups - 1);
        const int gx = min(base + kWin + j, groups - 1);  // look-ahead (threads j < U - 1)
        int kvr[kRows], kvx[kRows];
        const int sq_raw = row_seq[(size_t)gc * kRows];
        const int sqx_raw = row_seq[(size_t)gx * kRows];
        load_kv(gc, kvr);
        load_kv(gx, kvx);
        __builtin_amdgcn_sched_barrier(0);  // all 18 loads in flight before any is used
        const int gk_raw = group_kv(gc, kvr);
        const int gkx_raw = group_kv(gx, kvx);
        const int sq = in ? sq_raw : 0;
        s_sq[j] = sq;
        s_gk[j] = in ? gk_raw : 0;
        {  // look-ahead for units that straddle the window's end: threads j < U - 1
            // write slot kWin + j, the others the spare last slot (never read),
            // so no branch holds the look-ahead loads back
            const bool inx = j < U - 1 && base + kWin + j < groups;
            s_sq[kWin + min(j, U - 1)] = inx ? sqx_raw : 0;
            s_gk[kWin + min(j, U - 1)] = inx ? gkx_raw : 0;
        }
        __syncthreads();
        const int prev = j > 0 ? s_sq[j - 1] : c_sq;
        const bool new_run = in && (gi == 0 || sq != prev);
        int rs = block_scan_1024(new_run ? gi : -1, -1, s_tot, mx);
        if (rs < 0) rs = c_rs;
        const bool start = in && ((gi - rs) & (U - 1)) == 0;
        int c = 1, kv = s_gk[j];
#pragma unroll
        for (int k = 1; k < U; ++k)
            if (c == k && gi + k < groups && s_sq[j + k] == sq) {
                ++c;
                kv = max(kv, s_gk[j + k]);
            }
        const int w = U > 2 ? (c > 2 ? 4 : 3) : 1;
        const int n = (kv + pass - 1) / pass;
        const int lead = n > 0 ? kPieceCost : 0;
        const int work = start ? lead + w * n : 0;  // per kv head (every head has it)
        const int ui = block_scan_1024(start ? 1 : 0, 0, s_tot, add);
        const int wi = block_scan_1024(work, 0, s_tot, add);
        if (start) {
            const int o = c_units + ui - 1;
            const mfma::PagedUnit rec{gi, c, kv, c_work + wi - work + lead, n, w, o, 0};
            units[o] = rec;
            for (int k = 0; k < c; ++k) group_unit[gi + k] = rec;
        }
        if (j == kWin - 1) {  // window totals (inclusive scans at the last thread)
            s_carry[0] = ui;
            s_carry[1] = wi;
            s_carry[2] = rs;
            s_carry[3] = s_sq[min(groups - base, kWin) - 1];
        }
        __syncthreads();
        c_units += s_carry[0];
        c_work += s_carry[1];
        c_rs = s_carry[2];
        c_sq = s_carry[3];
        __syncthreads();  // before the next window rewrites s_sq and s_carry
    }
    if (j == 0) {
        units[c_units] = mfma::PagedUnit{0, 0, 0, c_work, 0, 1, c_units, 0};  // sentinel
        plan[0] = c_units;
        plan[1] = c_work;
    }
}

// ===========================================================================
// Decode over slot-mapped tokens: the reference's fused attention entries
// (src/cuda/tq_turbo_prod_kernels.cu:439-571, 650-671;
// src/cuda/tq_turbo_mse_kernels.cu:302-417, 459-479) for D = 128 and
// turbo_prod / turbo_mse pages.
//
// Flash-decoding split-K on a (split, kv head, row group) grid, 8 waves of
// 32-token chunks per workgroup, the same MFMA formulation as
// attn_mfma_split_kernel (QK: A = decoded K, B = the rotated query as fp16
// hi/lo columns; PV: A = P', B = decoded V), with a setup and a chunk loop
// cut to what the decode needs:
//  - one LDS lookup per K code byte returns two fp16 pairs: turbo_prod's
//    aK*K3 pair and its pair of residual signs (+-1; no VALU builds the sign
//    matrix), turbo_mse's hi and lo parts of aV*V4 (its V lookups read the
//    hi pair of the same entry);
//  - the tables are copied into LDS from compile-time constants while the
//    slots and codes are in flight (no per-entry arithmetic, no staging
//    pass);
//  - each wave rotates one query row and stores its fp16 hi and lo parts
//    straight into the B-operand layout: one barrier for the whole setup;
//  - P' = p * vs / aV enters the PV product as its fp16 hi part, or on the
//    lo columns as fp16(p * vs / aV - hi) of the exact product (three
//    mixed-precision ops per value pair and lane);
//  - per split and row the partial o[128] and (m, l) go to two arrays, the
//    (m, l) of one row contiguous over the splits, for
//    attn_decode_combine_kernel.
// ===========================================================================
namespace dec {
using namespace mfma;

// LDS layout of the tables (entries as decode_table_words describes) (32 copies of each entry, copy c at 4c; lane l
// reads copy l % 32, so a half-wave's random lookups hit distinct banks):
//   S table: byte 256b + 4c (the rows' upper halves unused: the table ends
//   below kOffK);
//   K table: byte kOffK + 256b + 4c (turbo_mse's V lookups read it too);
//   turbo_prod's V table: kOffK + 256b + 128 + 4c.
// A K lookup reads its S and K entries from one address register with
// offsets 0 and kOffK: no two-address LDS read reaches that pair (ds_read2
// spans up to 1020 bytes, ds_read2st64 multiples of 256), so each result
// goes straight into its MFMA operand registers.
constexpr int kOffK = 65520;
constexpr int kLutWords = (kOffK + 256 * 256) / 4;

// LDS address of copy (lane & 31) of entry `byte b of word` in a table of
// 256-byte entries at `base` (base = table + copy offset): v_perm puts the
// code byte in byte 1, and byte 1 of the base is added back.
__device__ __forceinline__ uint32_t lut_addr(uint32_t word, int b, uint32_t base) {
    return __builtin_amdgcn_perm(word, base, 0x03020000u | ((4u + b) << 8)) + (base & 0xFF00u);
}

// fp16 pair of x0 = a0 * b0, x1 = a1 * b1 for this lane's MFMA column: the
// hi parts fp16(x), or with lomask = ~0 the lo parts fp16(x - hi) of the
// exact products (v_fma_mix: one rounding to fp16).
__device__ __forceinline__ uint32_t hilo_pair(float a0, float b0, float a1, float b1,
                                              uint32_t lomask) {
    uint32_t h, r;
    asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,0,0]\n\t"
        "v_fma_mixhi_f16 %0, %3, %4, 0 op_sel_hi:[0,0,0]"
        : "=&v"(h)
        : "v"(a0), "v"(b0), "v"(a1), "v"(b1));
    const uint32_t m = h & lomask;
    asm("v_fma_mixlo_f16 %0, %1, %2, -%5 op_sel_hi:[0,0,1]\n\t"
        "v_fma_mixhi_f16 %0, %3, %4, -%5 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
        : "=&v"(r)
        : "v"(a0), "v"(b0), "v"(a1), "v"(b1), "v"(m));
    return r;
}

constexpr int kWaves = 8, kChunk = 32, kPass = kWaves * kChunk;
// Partial of (split, row): o[128] at po[(pid * 8 + r) * 128], (m, l) at
// pml[(item * 8 + r) * S + split] with pid = item * S + split and item =
// row group * H + kv head.
constexpr size_t kPartBytes = kRows * (128 * sizeof(float) + 2 * sizeof(float));

template <int SCH>
__global__ __launch_bounds__(64 * kWaves) void attn_decode_split_kernel(
    const uint16_t* __restrict__ query, const uint8_t* __restrict__ pool,
    const int32_t* __restrict__ slots, float* __restrict__ po, float2* __restrict__ pml,
    float inv, int num_queries, int num_kv_tokens, int tokens_per_split, int num_splits,
    PageGeom g) {
    constexpr bool PROD = SCH == kSchProd;
    static_assert(SCH == kSchProd || SCH == kSchMse, "turbo_prod or turbo_mse pages");
    // The decode tables (layout above); after the chunk loop the space holds
    // the waves' results for the merge.
    __shared__ __attribute__((aligned(256))) uint32_t lut[kLutWords];
    __shared__ uint4 bqs[4][64];  // QK B operand of k-step s for lane l
    __shared__ uint64_t tko[kWaves][kChunk], tvo[kWaves][kChunk];
    __shared__ float4 tsc[kWaves][kChunk];  // per token: K scale, residual scale, vs / aV, bias
    __shared__ float mm[kWaves][kRows], ml[kWaves][kRows];
    float(*mo)[kRows][128] = reinterpret_cast<float(*)[kRows][128]>(&lut[0]);
    static_assert(sizeof(float) * kWaves * kRows * 128 <= sizeof(lut), "merge space");

    int split, h, rg;
    if (gridDim.x == (unsigned)num_splits) {
        split = blockIdx.x;
        h = blockIdx.y;
        rg = blockIdx.z;
    } else {  // one dimension of splits x heads x row groups
        split = blockIdx.x % num_splits;
        const int hr = blockIdx.x / num_splits;
        h = hr % g.H;
        rg = hr / g.H;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, gq = lane >> 4;
    const int t_begin = split * tokens_per_split;
    const int t_end = min(num_kv_tokens, t_begin + tokens_per_split);
    // logit scale per unit ks (log2(e) / alpha folded at compile time: no run-time division)
    const float ck = inv * (PROD ? kLog2e / kAlphaK : kLog2e / kAlphaV);
    const float cr = inv * kLog2e;                                 // residual: ks * re
    constexpr float iav = 1.0f / kAlphaV;

    // 1. Loads, in the order they are needed: this wave's query row, the
    //    first chunk's slots, then the decode-table words.
    const int qrow = rg * kRows + w;
    const uint32_t qraw = *reinterpret_cast<const uint32_t*>(
        query + ((size_t)min(qrow, num_queries - 1) * g.H + h) * 128 + 2 * lane);
    int t0 = t_begin + w * kChunk;
    auto load_slot = [&](int t) -> int {
        return slots[max(min(t + (lane & (kChunk - 1)), t_end - 1), 0)];
    };
    const int slot0 = load_slot(t0);
    // 2. The chunk's codes and per-token scales.  slot -> cell offsets
    //    (exchanged through this wave's LDS rows) -> scale and code loads.
    //    Tokens past the range or with a negative slot read the first bytes
    //    of the query instead (always valid memory) and get bias -inf.
    struct Chunk {
        uint4 kw[2];     // K: tile tau, token 16 tau + i, bytes [16 gq, 16 gq + 16)
        uint32_t vw[8];  // V: k-index 8 gq + e (token below), dword i
        uint16_t ks, re, vs;
        bool valid;
    };
    const uint64_t dummy_off =
        (uint64_t)(reinterpret_cast<uintptr_t>(query) - reinterpret_cast<uintptr_t>(pool));
    auto fetch = [&](int tc, int slot, Chunk& c) {
        c.valid = tc + (lane & (kChunk - 1)) < t_end && slot >= 0;
        int page, tib;
        split_slot(c.valid ? slot : 0, g, page, tib);
        const uint64_t cell = (uint64_t)(tib * g.H + h);
        const uint64_t pb = (uint64_t)page * g.page_size;
        const uint64_t so = pb + cell * g.scale_stride;
        c.ks = ld_u16_nt(pool + (c.valid ? so + g.ks_off : dummy_off));
        c.vs = ld_u16_nt(pool + (c.valid ? so + g.vs_off : dummy_off + 2));
        c.re = PROD ? ld_u16_nt(pool + (c.valid ? so + g.kres_off : dummy_off + 4)) : (uint16_t)0;
        tko[w][lane & (kChunk - 1)] = c.valid ? pb + g.kc_off + cell * g.code_stride : dummy_off;
        tvo[w][lane & (kChunk - 1)] = c.valid ? pb + g.vc_off + cell * g.code_stride : dummy_off;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int tau = 0; tau < 2; ++tau) c.kw[tau] = ld_u4_nt(pool + (tko[w][16 * tau + i] + 16 * gq));
        // k-index 8 gq + e is token 4 gq + e (e < 4) or 16 + 4 gq + (e - 4)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int tok = e < 4 ? 4 * gq + e : 16 + 4 * gq + (e - 4);
            c.vw[e] = ld_u32_nt(pool + (tvo[w][tok] + 4 * i));
        }
    };
    Chunk cur;
    fetch(t0, slot0, cur);
    int slot_nx = load_slot(t0 + kPass);
    __builtin_amdgcn_sched_barrier(0);  // the code loads go out before any setup work

    // The tables' words, computed in registers while the codes are in flight
    // (no memory traffic; each 16-byte store writes four copies).
    const TableWords<PROD> tw = decode_table_words<PROD>(w, lane);
    // 3. This wave's query row: qrot = WHT(q * s) * inv, stored as fp16 hi
    //    and lo parts into the B operand (column 2w: hi, 2w + 1: lo; lane l
    //    holds d = 2l, 2l + 1: k-group l / 16, k-step (l / 4) % 4, halves
    //    2(l % 4), + 1 of the half8).
    {
        const float sh = (h & 1) ? -1.0f : 1.0f;
        float q0 = h2f(qraw & 0xffff) * sh, q1 = h2f(qraw >> 16) * (-sh);
        wht_pair<64>(q0, q1, lane);
        const bool live = qrow < num_queries;
        q0 = live ? q0 * inv : 0.0f;
        q1 = live ? q1 * inv : 0.0f;
        const uint32_t hi = pack_h2(q0, q1);
        const uint32_t lo = lo_pair(q0, q1, hi);
        uint32_t* b = reinterpret_cast<uint32_t*>(&bqs[(lane >> 2) & 3][16 * (lane >> 4) + 2 * w]);
        b[lane & 3] = hi;
        b[4 + (lane & 3)] = lo;  // the next lane's (column 2w + 1) half8
    }
    // 4. The decode tables.
    store_decode_tables<PROD>(lut, kOffK / 4, w, lane, tw);
    lds_barrier();
    half8 bq[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) bq[s] = __builtin_bit_cast(half8, bqs[s][lane]);

    // Lookup bases: copy lane % 32 of entry 0 of the S table (the K table
    // is kOffK above it; turbo_mse's V lookups read it that way), and of
    // turbo_prod's V table.
    const uint32_t basek = (uint32_t)reinterpret_cast<uintptr_t>((lds_u32*)&lut[lane & 31]);
    const uint32_t basev =
        PROD ? (uint32_t)reinterpret_cast<uintptr_t>((lds_u32*)&lut[kOffK / 4 + 32 + (lane & 31)])
             : basek;
    constexpr uint32_t offv = PROD ? 0u : (uint32_t)kOffK;
    const bool lo_col = (i & 1) != 0;
    const uint32_t lomask = lo_col ? 0xFFFFFFFFu : 0u;

    float m_run = kInitMax, l_run = 0.0f;
    f32x4 acc[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) acc[v] = (f32x4){0.f, 0.f, 0.f, 0.f};
    bool first = true;

    while (t0 < t_end) {  // wave-uniform
        {
            const float ks = h2f(cur.ks), vs = h2f(cur.vs), re = PROD ? h2f(cur.re) : 0.0f;
            const float4 sc = PROD ? make_float4(ks * ck, ks * re * cr, vs * iav, 0.0f)
                                   : make_float4(ks * ck, ks * ck * kLoScale, vs * iav, 0.0f);
            tsc[w][lane & (kChunk - 1)] = cur.valid ? sc : make_float4(0.f, 0.f, 0.f, -INFINITY);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        Chunk nxt;
        const int t1 = t0 + kPass;
        if (t1 < t_end) {  // codes of the next chunk, slots of the one after
            fetch(t1, slot_nx, nxt);
            slot_nx = load_slot(t1 + kPass);
        }
        // Per-token scales of this lane's logits (read before the lookups:
        // LDS reads complete in order).
        float4 scv[2][4];
#pragma unroll
        for (int tau = 0; tau < 2; ++tau)
#pragma unroll
            for (int e = 0; e < 4; ++e) scv[tau][e] = tsc[w][16 * tau + 4 * gq + e];
        // QK: every K lookup of the chunk issued before the first MFMA.
        half8 ka[2][4], kb[2][4];
#pragma unroll
        for (int tau = 0; tau < 2; ++tau) {
            const uint32_t wd[4] = {cur.kw[tau].x, cur.kw[tau].y, cur.kw[tau].z, cur.kw[tau].w};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                uint32_t e0[4], e1[4];  // K entries, S entries
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const uint32_t a = lut_addr(wd[s], b, basek);
                    e0[b] = *reinterpret_cast<const lds_u32*>(a + kOffK);
                    e1[b] = *reinterpret_cast<const lds_u32*>(a);
                }
                ka[tau][s] = as_h8(e0[0], e0[1], e0[2], e0[3]);
                kb[tau][s] = as_h8(e1[0], e1[1], e1[2], e1[3]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        f32x4 cb[2], cs[2];
#pragma unroll
        for (int tau = 0; tau < 2; ++tau) {
            cb[tau] = (f32x4){0.f, 0.f, 0.f, 0.f};
            cs[tau] = cb[tau];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                cb[tau] = mma(ka[tau][s], bq[s], cb[tau]);
                cs[tau] = mma(kb[tau][s], bq[s], cs[tau]);  // prod: residual signs; mse: lo parts
            }
        }
        // V lookups (B operands of PV), in flight during the softmax.
        uint32_t bv[8][4];  // [N-tile v = d - 8i][token pair]
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t we = cur.vw[2 * q], wo = cur.vw[2 * q + 1];
            const uint32_t lob = (we & 0x0F0F0F0Fu) | ((wo & 0x0F0F0F0Fu) << 4);
            const uint32_t hib = ((we >> 4) & 0x0F0F0F0Fu) | (wo & 0xF0F0F0F0u);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                bv[2 * b][q] = *reinterpret_cast<const lds_u32*>(lut_addr(lob, b, basev) + offv);
                bv[2 * b + 1][q] = *reinterpret_cast<const lds_u32*>(lut_addr(hib, b, basev) + offv);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // Logits (base 2) of tokens 16 tau + 4 gq + e; hi + lo columns summed.
        float lg[2][4];
        float mloc = -INFINITY;
#pragma unroll
        for (int tau = 0; tau < 2; ++tau)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float4 sc = scv[tau][e];
                const float sb = cb[tau][e] + quad_xor<1>(cb[tau][e]);
                const float sr = cs[tau][e] + quad_xor<1>(cs[tau][e]);
                lg[tau][e] = fmaf(sb, sc.x, fmaf(sr, sc.y, sc.w));
                mloc = fmaxf(mloc, lg[tau][e]);
            }
        mloc = lane_xor_reduce<16>(mloc, [](float x, float y) { return fmaxf(x, y); });
        mloc = lane_xor_reduce<32>(mloc, [](float x, float y) { return fmaxf(x, y); });
        // v_exp_f32 without denormal handling: arguments are <= 0 and a weight
        // below 2^-126 of the running maximum is negligible.
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = first ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        float lsum = 0.0f;
#pragma unroll
        for (int tau = 0; tau < 2; ++tau)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                lg[tau][e] = __builtin_amdgcn_exp2f(lg[tau][e] - m_new);
                lsum += lg[tau][e];
            }
        l_run = l_run * alpha + lsum;
        if (!first && __any(alpha != 1.0f)) {
            // acc lane (d, g) holds columns 4g .. 4g + 3 = rows 2g, 2g + 1
            const float a0 = __shfl(alpha, 4 * gq), a1 = __shfl(alpha, 4 * gq + 2);
#pragma unroll
            for (int v = 0; v < 8; ++v) {
                acc[v][0] *= a0;
                acc[v][1] *= a0;
                acc[v][2] *= a1;
                acc[v][3] *= a1;
            }
        }
        // PV: P' = p * vs / aV as this column's fp16 part; k-index 8 gq + e is
        // the logit of tile e / 4, element e % 4.
        const half8 ap = as_h8(hilo_pair(lg[0][0], scv[0][0].z, lg[0][1], scv[0][1].z, lomask),
                               hilo_pair(lg[0][2], scv[0][2].z, lg[0][3], scv[0][3].z, lomask),
                               hilo_pair(lg[1][0], scv[1][0].z, lg[1][1], scv[1][1].z, lomask),
                               hilo_pair(lg[1][2], scv[1][2].z, lg[1][3], scv[1][3].z, lomask));
#pragma unroll
        for (int v = 0; v < 8; ++v)
            acc[v] = mma(ap, as_h8(bv[v][0], bv[v][1], bv[v][2], bv[v][3]), acc[v]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        cur = nxt;
        t0 = t1;
        first = false;
    }

    // Wave results: l summed over the 4 lane groups of each column; o rows
    // from the hi + lo columns.  Then the waves are merged per row, the
    // inverse WHT and sign flip applied, and the partial written.
    {
        float l_tot = lane_xor_reduce<16>(l_run, [](float x, float y) { return x + y; });
        l_tot = lane_xor_reduce<32>(l_tot, [](float x, float y) { return x + y; });
        if (gq == 0 && !lo_col) {
            mm[w][i >> 1] = m_run;
            ml[w][i >> 1] = l_tot;
        }
    }
    lds_barrier();  // every wave is done with the tables mo overwrites
#pragma unroll
    for (int v = 0; v < 8; ++v) {
        mo[w][2 * gq][8 * i + v] = acc[v][0] + acc[v][1];
        mo[w][2 * gq + 1][8 * i + v] = acc[v][2] + acc[v][3];
    }
    lds_barrier();
    const int r = w;  // this wave's row of the group
    if (rg * kRows + r >= num_queries) return;  // wave-uniform, after the last barrier
    float M = mm[0][r];
#pragma unroll
    for (int u = 1; u < kWaves; ++u) M = fmaxf(M, mm[u][r]);
    float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int u = 0; u < kWaves; ++u) {
        const float wt = __builtin_amdgcn_exp2f(mm[u][r] - M);  // (argument <= 0)
        const float2 ov = *reinterpret_cast<const float2*>(&mo[u][r][2 * lane]);
        L += ml[u][r] * wt;
        o0 += ov.x * wt;
        o1 += ov.y * wt;
    }
    wht_pair<64>(o0, o1, lane);
    const float s0 = (h & 1) ? -inv : inv;
    const size_t item = (size_t)rg * g.H + h;
    const size_t pid = item * num_splits + split;
    *reinterpret_cast<float2*>(po + (pid * kRows + r) * 128 + 2 * lane) = make_float2(o0 * s0, o1 * -s0);
    if (lane == 0) pml[(item * kRows + r) * num_splits + split] = make_float2(M, L);
}

// Sum of the split partials of one output row (q, h): o = sum_s 2^(m_s - M)
// o_s / sum_s 2^(m_s - M) l_s.  One wave per (row, 8-element slice of d):
// lane = 8 split groups x 8 elements; group j takes splits j, j + 8, ..., 16
// at a time (every load of a batch in flight together), merges them with a
// running maximum, then the groups are merged across lanes (no LDS, no
// barrier).  The 4 slices of one 128-byte line of the partials run on one
// XCD (block b on XCD b % 8), so three of them find the line in that XCD's
// L2.
__global__ __launch_bounds__(64) void attn_decode_combine_kernel(
    const float* __restrict__ po, const float2* __restrict__ pml, uint16_t* __restrict__ output,
    int H, int rows, int S) {
    using namespace mfma;
    const int b = blockIdx.x;
    const int xcd = b & 7, m = b >> 3;
    const int p = (m >> 2) * 8 + xcd;  // (row, line) pair
    const int row = p >> 2;
    if (row >= rows) return;
    const int t = threadIdx.x, dd = t & 7, grp = t >> 3;
    const int d = 32 * (p & 3) + 8 * (m & 3) + dd;
    const int q = row / H, h = row - q * H;
    const int rg = q / kRows, r = q % kRows;
    const size_t item = (size_t)rg * H + h;
    const float2* mlr = pml + (item * kRows + r) * S;
    const float* orow = po + (item * S * kRows + r) * 128 + d;  // split s: + s * kRows * 128
    constexpr int kB = 16;
    float M = kInitMax, L = 0.f, A = 0.f;
    for (int base = grp; base < S; base += 8 * kB) {
        float pm[kB], pl[kB], pv[kB];
#pragma unroll
        for (int k = 0; k < kB; ++k) {
            const int s = base + 8 * k;
            const int sc = s < S ? s : base;
            const float2 v = mlr[sc];
            pm[k] = s < S ? v.x : kInitMax;
            pl[k] = v.y;
            pv[k] = orow[(size_t)sc * kRows * 128];
        }
        float mb = M;
#pragma unroll
        for (int k = 0; k < kB; ++k) mb = fmaxf(mb, pm[k]);
        // v_exp_f32 without denormal handling: arguments are <= 0 and a weight
        // below 2^-126 of the largest is negligible.
        const float sc = __builtin_amdgcn_exp2f(M - mb);
        L *= sc;
        A *= sc;
#pragma unroll
        for (int k = 0; k < kB; ++k) {
            const float wt = __builtin_amdgcn_exp2f(pm[k] - mb);
            L += pl[k] * wt;
            A += pv[k] * wt;
        }
        M = mb;
    }
    auto merge = [&](float Mp, float Lp, float Ap) {
        const float mn = fmaxf(M, Mp);
        const float a = __builtin_amdgcn_exp2f(M - mn), c = __builtin_amdgcn_exp2f(Mp - mn);
        L = L * a + Lp * c;
        A = A * a + Ap * c;
        M = mn;
    };
    merge(lane_xor<8>(M), lane_xor<8>(L), lane_xor<8>(A));
    merge(lane_xor<16>(M), lane_xor<16>(L), lane_xor<16>(A));
    merge(lane_xor<32>(M), lane_xor<32>(L), lane_xor<32>(A));
    if (t < 8) output[(size_t)row * 128 + d] = f2h(L > 0.f ? A / L : A);
}

}  // namespace dec

// New-token positions (row groups of one sequence) per paged workgroup.
#ifndef TQ_PAGED_POSITIONS
#define TQ_PAGED_POSITIONS 4
#endif
constexpr int kPagedPositions = TQ_PAGED_POSITIONS;
// Paged steps: work segments (workgroups) per CU.
#ifndef TQ_PAGED_SEGMENTS_PER_CU
#define TQ_PAGED_SEGMENTS_PER_CU 1
#endif
constexpr int kPagedSegmentsPerCU = TQ_PAGED_SEGMENTS_PER_CU;

// Split kernel shape: tokens per wave iteration and waves per workgroup.
#ifndef TQ_SPLIT_CHUNK
#define TQ_SPLIT_CHUNK 32
#endif
#ifndef TQ_SPLIT_WAVES
#define TQ_SPLIT_WAVES 8
#endif
#ifndef TQ_SPLIT_MIN_TOKENS
#define TQ_SPLIT_MIN_TOKENS 256
#endif
#ifndef TQ_SPLIT_BLOCKS_PER_CU
#define TQ_SPLIT_BLOCKS_PER_CU 2
#endif
constexpr int kSplitChunk = TQ_SPLIT_CHUNK, kSplitWaves = TQ_SPLIT_WAVES;
constexpr int kSplitMinTokens = TQ_SPLIT_MIN_TOKENS, kSplitBlocksPerCU = TQ_SPLIT_BLOCKS_PER_CU;

bool mfma_attention_ok(const PageGeom& g, const void* pool) {
    const auto al = [](uint64_t v, uint64_t a) { return (v & (a - 1)) == 0; };
    return g.D == 128 && g.code_stride == 64 && al(g.page_size, 16) && al(g.kc_off, 16) &&
           al(g.vc_off, 4) && al(reinterpret_cast<uintptr_t>(pool), 16);
}

}  // namespace

#define TQ_DISPATCH_D(D_, ...)                                                 \
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

namespace {
// The MFMA split-K attention over slot-mapped tokens: split + combine launches.
template <int SCH>
void launch_mfma_attention(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                           uint16_t* output, const PageGeom& g, int num_queries,
                           int num_kv_tokens, float inv, hipStream_t stream, const char* split_name,
                           const char* combine_name, const Scratch& scratch = Scratch{}) {
    using namespace mfma;
    const int rows = num_queries * g.H;
    const int row_groups = (num_queries + kRows - 1) / kRows;
    const int heads = g.H * row_groups;
    // One 256-token split per workgroup, or longer splits once there are
    // more than ~2 workgroups per CU.
    const int max_splits = std::max(1, (num_kv_tokens + kSplitMinTokens - 1) / kSplitMinTokens);
    const int want = std::max(1, (kSplitBlocksPerCU * num_cus() + heads - 1) / heads);
    int splits = std::min(std::min(max_splits, want), 1024);
    const int tps = num_kv_tokens > 0 ? (num_kv_tokens + splits - 1) / splits : 0;
    if (tps > 0) splits = (num_kv_tokens + tps - 1) / tps;
    const size_t blocks = (size_t)splits * heads;
    float* ws = static_cast<float*>(
        scratch.get(stream, blocks * kRows * kPartStride * sizeof(float), split_name));
    constexpr int kCH = kSplitChunk, kNW = kSplitWaves;
    const PagedRows none{};
    constexpr int kMaxGridYZ = 65535;
    const dim3 combine_grid = num_queries <= kMaxGridYZ && g.H <= kMaxGridYZ
                                  ? dim3(4, g.H, num_queries)
                                  : dim3(4 * rows);
    if (num_kv_tokens == 0) {  // no partials: the combine writes the zero output
        hipLaunchKernelGGL(attn_mfma_combine_kernel, combine_grid, dim3(256), 0, stream, ws,
                           output, g.H, 0);
        check_launch(combine_name);
        return;
    }
    const dim3 grid = row_groups <= kMaxGridYZ && g.H <= kMaxGridYZ
                          ? dim3(splits, g.H, row_groups)
                          : dim3((unsigned)blocks);
    hipLaunchKernelGGL((attn_mfma_split_kernel<SCH, kCH, kNW, false>), grid, dim3(64 * kNW), 0,
                       stream, query, pool, slots, ws, inv, num_queries, num_kv_tokens, tps, splits,
                       g, none);
    check_launch(split_name);
    if (splits <= kItemCombineMaxSplits)
        hipLaunchKernelGGL(attn_mfma_combine_items_kernel, dim3(heads), dim3(256), 0, stream,
                           ws, output, g.H, splits, num_queries);
    else
        hipLaunchKernelGGL(attn_mfma_combine_kernel, combine_grid, dim3(256), 0, stream, ws,
                           output, g.H, splits);
    check_launch(combine_name);
}

// The slot-mapped decode (turbo_prod, turbo_mse; D = 128): split + combine.
template <int SCH>
void launch_decode_attention(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                             uint16_t* output, const PageGeom& g, int num_queries,
                             int num_kv_tokens, float inv, hipStream_t stream,
                             const char* split_name, const char* combine_name,
                             const Scratch& scratch) {
    using namespace mfma;
    const int rows = num_queries * g.H;
    const int row_groups = (num_queries + kRows - 1) / kRows;
    const int heads = g.H * row_groups;
    // One 256-token split per workgroup, or longer splits once there are
    // more than ~2 workgroups per CU.
    const int max_splits = std::max(1, (num_kv_tokens + kSplitMinTokens - 1) / kSplitMinTokens);
    const int want = std::max(1, (kSplitBlocksPerCU * num_cus() + heads - 1) / heads);
    int splits = std::min(std::min(max_splits, want), 1024);
    const int tps = num_kv_tokens > 0 ? (num_kv_tokens + splits - 1) / splits : 0;
    if (tps > 0) splits = (num_kv_tokens + tps - 1) / tps;
    // The combine: 32 blocks per pair of output rows (8-element slices).
    const long long combine_blocks = ((long long)rows + 1) / 2 * 32;
    if (combine_blocks > INT32_MAX) throw Error(std::string(combine_name) + ": too many query rows");
    const size_t blocks = (size_t)splits * heads;
    char* ws = static_cast<char*>(scratch.get(stream, blocks * dec::kPartBytes, split_name));
    float* po = reinterpret_cast<float*>(ws);
    float2* pml = reinterpret_cast<float2*>(ws + blocks * kRows * 128 * sizeof(float));
    if (num_kv_tokens > 0) {
        constexpr int kMaxGridYZ = 65535;
        const dim3 grid = row_groups <= kMaxGridYZ && g.H <= kMaxGridYZ
                              ? dim3(splits, g.H, row_groups)
                              : dim3((unsigned)blocks);
        hipLaunchKernelGGL((dec::attn_decode_split_kernel<SCH>), grid, dim3(64 * dec::kWaves), 0,
                           stream, query, pool, slots, po, pml, inv, num_queries, num_kv_tokens,
                           tps, splits, g);
        check_launch(split_name);
    }
    // (no partials for an empty context: the combine writes zeros)
    hipLaunchKernelGGL(dec::attn_decode_combine_kernel, dim3((unsigned)combine_blocks), dim3(64),
                       0, stream, po, pml, output, g.H, rows, num_kv_tokens > 0 ? splits : 0);
    check_launch(combine_name);
}

// The generic split-K decode (attn_partial_kernel + attn_combine_kernel, any
// head_dim and page geometry): one wave per (split, row), enough waves to
// cover the chip several times, at least 32 tokens per split.
struct GenericSplit {
    int splits, tps;
    size_t ws_bytes;
};
GenericSplit generic_split(int rows, int max_tokens, int D) {
    int splits = (2048 + rows - 1) / rows;
    splits = std::min(splits, std::max(1, (max_tokens + 31) / 32));
    splits = std::max(splits, 1);
    const int tps = max_tokens > 0 ? (max_tokens + splits - 1) / splits : 0;
    if (tps > 0) splits = (max_tokens + tps - 1) / tps;
    return {splits, tps, (size_t)splits * rows * (D + 2) * sizeof(float)};
}
template <class Tok>
void launch_generic_attention(Scheme s, const uint16_t* query, const uint8_t* pool, Tok tok,
                              uint16_t* output, const PageGeom& g, int rows,
                              const GenericSplit& sp, float* ws, hipStream_t stream,
                              const char* name) {
    if ((long long)sp.splits * rows > INT32_MAX)
        throw Error(std::string(name) + ": too many query rows");
    const float inv = inv_sqrt_d(g.D);
    const dim3 grid((unsigned)(sp.splits * rows));
    if (s == Scheme::Prod) {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL((attn_partial_kernel<kD, true, Tok>), grid, dim3(64),
                                              0, stream, query, pool, tok, ws, g, rows, sp.tps,
                                              sp.splits, inv));
    } else {
        TQ_DISPATCH_D(g.D, hipLaunchKernelGGL((attn_partial_kernel<kD, false, Tok>), grid, dim3(64),
                                              0, stream, query, pool, tok, ws, g, rows, sp.tps,
                                              sp.splits, inv));
    }
    check_launch((std::string(name) + "_partial").c_str());
    TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(attn_combine_kernel<kD>, dim3(rows), dim3(64), 0,
                                          stream, ws, output, g, rows, sp.splits, inv));
    check_launch((std::string(name) + "_combine").c_str());
}
}  // namespace

void launch_attention(Scheme s, const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                      uint16_t* output, const PageGeom& g, int num_queries, int num_kv_tokens,
                      hipStream_t stream, const Scratch& scratch) {
    const int rows = num_queries * g.H;
    if (rows <= 0) return;
    const float inv = inv_sqrt_d(g.D);
    if (mfma_attention_ok(g, pool)) {
        if (s == Scheme::Prod)
            launch_decode_attention<mfma::kSchProd>(query, pool, slots, output, g, num_queries,
                                                    num_kv_tokens, inv, stream,
                                                    "turbo_prod_fused_attn_split",
                                                    "turbo_prod_fused_attn_combine", scratch);
        else
            launch_decode_attention<mfma::kSchMse>(query, pool, slots, output, g, num_queries,
                                                   num_kv_tokens, inv, stream,
                                                   "turbo_mse_fused_attn_split",
                                                   "turbo_mse_fused_attn_combine", scratch);
        return;
    }
    const GenericSplit sp = generic_split(rows, num_kv_tokens, g.D);
    const bool prod = s == Scheme::Prod;
    float* ws = static_cast<float*>(scratch.get(
        stream, sp.ws_bytes, prod ? "turbo_prod_fused_attn_partial" : "turbo_mse_fused_attn_partial"));
    launch_generic_attention(s, query, pool, SlotTokens{slots, num_kv_tokens}, output, g, rows, sp,
                             ws, stream, prod ? "turbo_prod_fused_attn" : "turbo_mse_fused_attn");
}

void launch_paged_attention(Scheme s, const uint16_t* query, const uint8_t* pool,
                            const int32_t* block_tables, int max_blocks, const int32_t* row_seq,
                            const int32_t* row_kv_len, uint16_t* output, const PageGeom& g,
                            int num_rows, int max_kv_len, hipStream_t stream) {
    const int rows = num_rows * g.H;
    if (rows <= 0) return;
    const bool prod = s == Scheme::Prod;
    // Bytes from a page's start that a cell's loads reach (the matrix-core
    // kernel addresses them as 32-bit offsets, and masked tokens read a spare
    // region of this size).
    const uint64_t cells = (uint64_t)g.block_size * (uint64_t)g.H;
    const uint64_t extent =
        std::max({g.page_size, std::max({g.ks_off, g.vs_off, g.kres_off}) + cells * g.scale_stride,
                  std::max(g.kc_off, g.vc_off) + cells * g.code_stride});
    if (!mfma_attention_ok(g, pool) || extent > 0xFFFFFFFFu) {
        // Other head_dims and unaligned pages: the generic split-K decode, its
        // rows reading their tokens through the block table.
        const GenericSplit sp = generic_split(rows, std::max(max_kv_len, 0), g.D);
        float* ws = static_cast<float*>(workspace(stream, sp.ws_bytes));
        launch_generic_attention(
            s, query, pool,
            PagedTokens{block_tables, row_seq, row_kv_len, max_blocks, std::max(max_kv_len, 0)},
            output, g, rows, sp, ws, stream,
            prod ? "turbo_prod_paged_attn" : "turbo_mse_paged_attn");
        return;
    }
    using namespace mfma;
    const float inv = inv_sqrt_d(g.D);
    const int row_groups = (num_rows + kRows - 1) / kRows;
    const int heads = g.H * row_groups;
    // The plan gives every kv head the same work (each unit's passes over
    // its kv length), split into Gh equal segments per head, one workgroup
    // each: G = H * Gh workgroups, Gh a multiple of 8 (the kernel's XCD
    // mapping).
    constexpr int kPass = kSplitChunk * kSplitWaves;
    const int Gh = 8 * ((kPagedSegmentsPerCU * num_cus() + 8 * g.H - 1) / (8 * g.H));
    const int G = Gh * g.H;
    // The plan counts each kv head's work in int32: at most
    // 4 * ceil(max_kv_len / kPass) + kPieceCost per row group (every head has
    // the same).
    if ((long long)row_groups *
            (4LL * ((std::max(max_kv_len, 0) + kPass - 1) / kPass) + kPieceCost) >
        INT32_MAX)
        throw Error("paged attention: too many rows for this max_kv_len");
    // Workspace: the partials (slot (unit + segment) * H + head: fewer than
    // (row_groups + Gh) * H = heads + G slots of kPagedPositions positions),
    // then the plan: the units and a
    // sentinel, each row group's unit, the unit count and total work.
    const size_t part_bytes =
        ((size_t)heads + G) * kPagedPositions * kRows * kPartStride * sizeof(float);
    const size_t unit_bytes = (2 * (size_t)row_groups + 1) * sizeof(PagedUnit);
    const size_t spare_at = (part_bytes + unit_bytes + 4 * sizeof(int32_t) + 255) & ~(size_t)255;
    char* wsb = static_cast<char*>(workspace(stream, spare_at + extent));
    float* ws = reinterpret_cast<float*>(wsb);
    PagedUnit* units = reinterpret_cast<PagedUnit*>(wsb + part_bytes);
    PagedUnit* group_unit = units + row_groups + 1;
    int32_t* plan = reinterpret_cast<int32_t*>(wsb + part_bytes + unit_bytes);
    const PagedRows pr{block_tables, row_seq,    row_kv_len, max_blocks, units, group_unit, plan,
                       reinterpret_cast<const uint8_t*>(wsb + spare_at)};
    constexpr int kCH = kSplitChunk, kNW = kSplitWaves;
    hipLaunchKernelGGL(paged_plan_kernel<kPagedPositions>, dim3(1), dim3(1024), 0, stream, row_seq,
                       row_kv_len, num_rows, row_groups, kPass, std::max(max_kv_len, 0), units,
                       group_unit, plan);
    check_launch(prod ? "turbo_prod_paged_attn_plan" : "turbo_mse_paged_attn_plan");
    if (max_kv_len > 0) {
        if (prod)
            hipLaunchKernelGGL((attn_mfma_split_kernel<kSchProd, kCH, kNW, true, kPagedPositions>),
                               dim3(G), dim3(64 * kNW), 0, stream, query, pool, nullptr, ws, inv,
                               num_rows, max_kv_len, 0, 0, g, pr);
        else
            hipLaunchKernelGGL((attn_mfma_split_kernel<kSchMse, kCH, kNW, true, kPagedPositions>),
                               dim3(G), dim3(64 * kNW), 0, stream, query, pool, nullptr, ws, inv,
                               num_rows, max_kv_len, 0, 0, g, pr);
        check_launch(prod ? "turbo_prod_paged_attn_split" : "turbo_mse_paged_attn_split");
    }
    hipLaunchKernelGGL(attn_paged_combine_kernel, dim3(heads), dim3(256), 0, stream, ws, output,
                       g.H, num_rows, Gh, kPagedPositions, kPass, pr);
    check_launch(prod ? "turbo_prod_paged_attn_combine" : "turbo_mse_paged_attn_combine");
}

bool launch_qjl_mfma_attention(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                               uint16_t* output, const QjlGeom& q, int num_queries,
                               int num_kv_tokens, hipStream_t stream) {
    const auto al = [](uint64_t v, uint64_t a) { return (v & (a - 1)) == 0; };
    if (!(q.D == 128 && q.k1_bytes == 16 && q.v4_bytes == 64 && al(q.page_size, 4) &&
          al(q.k1_off, 4) && al(q.v4_off, 4) && al(q.ks_off, 2) && al(q.vs_off, 2) &&
          al(reinterpret_cast<uintptr_t>(pool), 16)))
        return false;
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
    launch_mfma_attention<mfma::kSchQjl>(query, pool, slots, output, g, num_queries,
                                         num_kv_tokens, inv_sqrt_d(q.D), stream,
                                         "qjl_fused_attn_split", "qjl_fused_attn_combine");
    return true;
}

void launch_logits(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                   float* logits, const PageGeom& g, int num_queries, int num_kv_tokens,
                   hipStream_t stream) {
    const int rows = num_queries * g.H;
    if (rows <= 0 || num_kv_tokens <= 0) return;
    const int tiles = (num_kv_tokens + 255) / 256;
    const float inv = inv_sqrt_d(g.D);
    const int row_groups = (num_queries + 7) / 8;
    if (g.D == 128 && g.code_stride == 64 && (g.kc_off & 3) == 0 && (g.page_size & 3) == 0 &&
        (g.ks_off & 1) == 0 && (g.kres_off & 1) == 0 &&
        (reinterpret_cast<uintptr_t>(pool) & 3) == 0 && g.H <= 65535 && row_groups <= 65535 &&
        g.page_size <= 0xFFFFFFFFull) {
        const bool vec = (num_kv_tokens & 3) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0;
        const dim3 grid((num_kv_tokens + lgt::kTokens - 1) / lgt::kTokens, g.H, row_groups);
        const dim3 block(64 * lgt::kWaves);
        if (vec)
            hipLaunchKernelGGL((lgt::prod_logits_mfma_kernel<true>), grid, block, 0, stream, query,
                               pool, slots, logits, g, num_queries, num_kv_tokens, inv);
        else
            hipLaunchKernelGGL((lgt::prod_logits_mfma_kernel<false>), grid, block, 0, stream, query,
                               pool, slots, logits, g, num_queries, num_kv_tokens, inv);
        check_launch("turbo_prod_fused_attention_logits_kernel");
        return;
    }
    TQ_DISPATCH_D(g.D, hipLaunchKernelGGL(prod_logits_kernel<kD>, dim3(rows * tiles), dim3(256),
                                          0, stream, query, pool, slots, logits, g,
                                          num_kv_tokens, tiles, inv));
    check_launch("turbo_prod_fused_attention_logits_kernel");
}

}  // namespace tq

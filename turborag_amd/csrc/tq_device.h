// tq_device.h — device-side building blocks for the gfx950 kernels.
//
// Row convention: one (token, head) vector of D fp32 values ("row") is held by
// D/2 consecutive lanes of a wave64, lane j owning elements 2j and 2j+1.  With
// that assignment the reference's butterfly (len = 1 first, then 2, 4, ...)
// is: stage 1 in registers, stage len >= 2 an xor-exchange with lane
// j ^ (len/2); and the reference's shared-memory halving tree
// r[i] += r[i + s] is an xor-butterfly over lanes followed by r0 + r1.  Both
// reproduce the reference's float operation order exactly, so results are
// bit-identical to it (fp32 add is commutative; every lane of an xor pair
// computes the same sum).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "tq_internal.h"

namespace tq {
namespace dev {

// Codebooks: src/cuda/tq_turbo_prod_kernels.cu:26-37 (K3 3-bit Lloyd-Max,
// V4 4-bit) and src/cuda/tq_turbo_mse_kernels.cu:24-29 (turbo_mse = V4).
__device__ constexpr float kK3[8] = {-2.1513f, -1.34326f, -0.755526f, -0.244919f,
                                     0.244919f, 0.755526f, 1.34326f,  2.1513f};
__device__ constexpr float kV4[16] = {-2.7326f, -2.0690f, -1.6180f, -1.2562f,
                                      -0.9423f, -0.6568f, -0.3880f, -0.1284f,
                                      0.1284f,  0.3880f,  0.6568f,  0.9423f,
                                      1.2562f,  1.6180f,  2.0690f,  2.7326f};

constexpr float kMinRMS = 1e-8f;  // include/tq_shared_device.cuh:9

// t[idx] for a runtime idx, built from immediates (v_cndmask chain): no
// memory access, so it never waits behind outstanding global loads (the
// vector-memory counter is in order).
template <int N>
__device__ __forceinline__ float pick(const float (&t)[N], int idx) {
    float r = t[0];
#pragma unroll
    for (int k = 1; k < N; ++k) r = (idx == k) ? t[k] : r;
    return r;
}

// A float in LDS addressed by its 32-bit LDS byte offset.
typedef __attribute__((address_space(3))) float lds_float;
typedef __attribute__((address_space(3))) uint32_t lds_u32;

__device__ __forceinline__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}
// fp32 -> fp16, RNE (v_cvt_f16_f32).  The empty asm pins f as a rounded fp32
// register value: without it the backend folds fp16(a * b) into
// v_fma_mixlo_f16(a, b, 0), which rounds a*b once to fp16 (not fp32 then
// fp16, as the reference does) and turns a -0 product into +0.
__device__ __forceinline__ uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    return __half_as_ushort(__float2half(f));
}

// The reference's sign_flip(i, h) (tq_turbo_prod_kernels.cu:19-23) has bit 0
// of ((h*2654435761) ^ (i*1103515245 + 12345)) = 1 ^ ((i ^ h) & 1), i.e. it
// is exactly (-1)^(i+h).
__device__ __forceinline__ float sign_of(int i, int h) { return ((i ^ h) & 1) ? -1.0f : 1.0f; }

__device__ __forceinline__ float clamp_ref(float x, float lo, float hi) {
    return x < lo ? lo : (x > hi ? hi : x);
}

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }

// Two fp32 -> packed fp16x2 (RNE each, v_cvt_pk_f16_f32), low half = a.  Same
// fp32 pinning as f2h.
__device__ __forceinline__ uint32_t f2h2(float a, float b) {
    typedef float f2v __attribute__((ext_vector_type(2)));
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    asm volatile("" : "+v"(a), "+v"(b));
    const h2v h = __builtin_convertvector((f2v){a, b}, h2v);
    return __builtin_bit_cast(uint32_t, h);
}

// Lane exchange inside a quad through DPP (a VALU op, no LDS traffic):
// quad_perm(1,0,3,2) = xor 1, quad_perm(2,3,0,1) = xor 2.
template <int MASK>
__device__ __forceinline__ float quad_xor(float v) {
    static_assert(MASK == 1 || MASK == 2, "quad_xor: mask 1 or 2");
    constexpr int ctrl = MASK == 1 ? 0xB1 : 0x4E;
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, true));
}

// v of lane (this lane) ^ M across a full wave64, without LDS: DPP quad
// permutes for M = 1, 2; half-row mirror then quad reverse for 4; row rotate
// by 8 for 8; the gfx950 permlane16 / permlane32 swaps for 16 and 32.  Every
// lane of the wave must be active (the DPP reads use bound_ctrl).
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
    const int x = __float_as_int(v);
    if constexpr (M == 1 || M == 2) {
        return quad_xor<M>(v);
    } else if constexpr (M == 4) {
        const int t = __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, true);  // row_half_mirror
        return __int_as_float(__builtin_amdgcn_mov_dpp(t, 0x1B, 0xF, 0xF, true));  // quad 3210
    } else if constexpr (M == 8) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true));  // row_ror:8
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
        return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
    } else {
        static_assert(M == 32, "lane_xor: M in 1..32");
        const auto r = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
        return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
    }
}

// op(v, lane_xor<M>(v)) for a symmetric op (max, +).  M = 16, 32: a
// permlane swap of v with itself leaves v's even rows (halves) in one result
// and its odd rows in the other, each duplicated, so op over the two is the
// reduction in every lane: one swap, no lane select.
template <int M, class Op>
__device__ __forceinline__ float lane_xor_reduce(float v, Op op) {
    const unsigned x = __float_as_uint(v);
    if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
    } else if constexpr (M == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
    } else {
        return op(v, lane_xor<M>(v));
    }
}

// lane_xor for an m known after loop unrolling.
__device__ __forceinline__ float xor_lane(float v, int m) {
    switch (m) {
        case 1: return lane_xor<1>(v);
        case 2: return lane_xor<2>(v);
        case 4: return lane_xor<4>(v);
        case 8: return lane_xor<8>(v);
        case 16: return lane_xor<16>(v);
        default: return lane_xor<32>(v);
    }
}

// In-place WHT of a row held two-per-lane (lane index j within its row).
template <int L>
__device__ __forceinline__ void wht_pair(float& x0, float& x1, int j) {
    const float a = x0 + x1, b = x0 - x1;
    x0 = a;
    x1 = b;
#pragma unroll
    for (int m = 1; m < L; m <<= 1) {
        const float p0 = xor_lane(x0, m), p1 = xor_lane(x1, m);
        const bool lower = (j & m) == 0;
        x0 = lower ? x0 + p0 : p0 - x0;
        x1 = lower ? x1 + p1 : p1 - x1;
    }
}

// Halving tree over the row (strides D/2 ... 1); every lane gets r[0].
template <int L>
__device__ __forceinline__ float tree_pair(float r0, float r1) {
#pragma unroll
    for (int m = L / 2; m >= 1; m >>= 1) {
        r0 += xor_lane(r0, m);
        r1 += xor_lane(r1, m);
    }
    return r0 + r1;
}

// Halving tree over one value per lane (the turbo_mse pair sums).
template <int L>
__device__ __forceinline__ float tree_one(float r) {
#pragma unroll
    for (int m = L / 2; m >= 1; m >>= 1) r += xor_lane(r, m);
    return r;
}

template <int L>
__device__ __forceinline__ float sum_lanes(float r) {
    return tree_one<L>(r);
}

template <int L>
__device__ __forceinline__ float max_lanes(float r) {
#pragma unroll
    for (int m = L / 2; m >= 1; m >>= 1) r = fmaxf(r, xor_lane(r, m));
    return r;
}

// nearest_k3_idx / nearest_v4_idx (:39-59): first minimum of fp32 |x - c|.
__device__ __forceinline__ int nearest_k3(float x, float& level) {
    int best = 0;
    float bd = fabsf(x - kK3[0]);
    level = kK3[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) {
        const float d = fabsf(x - kK3[i]);
        if (d < bd) {
            bd = d;
            best = i;
            level = kK3[i];
        }
    }
    return best;
}

__device__ __forceinline__ int nearest_v4(float x) {
    int best = 0;
    float bd = fabsf(x - kV4[0]);
#pragma unroll
    for (int i = 1; i < 16; ++i) {
        const float d = fabsf(x - kV4[i]);
        if (d < bd) {
            bd = d;
            best = i;
        }
    }
    return best;
}

// Decision thresholds of the nearest-level scans.  For neighbouring levels
// a < b, closer(x) = fp32 |x - b| < fp32 |x - a| is false up to a and true
// from b on, and monotone in between (fp32 subtraction rounds monotonically),
// so on the clamped domain it is x >= T for T = the smallest float with
// closer(T).  The levels are sorted and at least 0.25 apart, far above the
// fp32 spacing of the distances, so the distances fall strictly up to the
// first minimum and rise after it: the index the reference's strict '<' scan
// returns is the number of strict decreases, #{i : x >= T_i}.  The T_i are
// computed here at compile time by bisection over floats with the same fp32
// operations.
namespace thr {
constexpr float cabs(float v) { return v < 0.0f ? -v : v; }
constexpr bool closer(float x, float a, float b) { return cabs(x - b) < cabs(x - a); }
// No float lies strictly between lo < hi exactly when their rounded midpoint
// is lo or hi.
constexpr bool adjacent(float lo, float hi) {
    return (lo + hi) * 0.5f == lo || (lo + hi) * 0.5f == hi;
}
template <int N>
struct Table {
    float t[N];      // t[i]: smallest float with closer(., c[i-1], c[i]); t[0] unused
    float below[N];  // the float just below t[i]
};
// Bisection keeps closer(lo) false and closer(hi) true until they are
// adjacent floats.
template <int N>
constexpr Table<N> thresholds(const float (&c)[N]) {
    Table<N> r{};
    for (int i = 1; i < N; ++i) {
        float lo = c[i - 1], hi = c[i];
        while (!adjacent(lo, hi)) {
            const float m = (lo + hi) * 0.5f;
            if (closer(m, c[i - 1], c[i]))
                hi = m;
            else
                lo = m;
        }
        r.t[i] = hi;
        r.below[i] = lo;
    }
    return r;
}
template <int N>
constexpr bool well_formed(const float (&c)[N], const Table<N>& T) {
    for (int i = 1; i < N; ++i) {
        if (!(c[i] - c[i - 1] >= 0.25f)) return false;  // the spacing the argument needs
        if (!(T.t[i] > c[i - 1] && T.t[i] <= c[i])) return false;
        if (!closer(T.t[i], c[i - 1], c[i]) || closer(T.below[i], c[i - 1], c[i])) return false;
        if (!(T.below[i] < T.t[i]) || !adjacent(T.below[i], T.t[i])) return false;
    }
    return true;
}
}  // namespace thr

__device__ constexpr thr::Table<8> kK3T = thr::thresholds(kK3);
__device__ constexpr thr::Table<16> kV4T = thr::thresholds(kV4);
static_assert(thr::well_formed(kK3, kK3T) && thr::well_formed(kV4, kV4T),
              "codebook thresholds");

// Grid form of the searches.  A cell g = (int)RN(8x + off) (8x is exact, so
// fma and mul-then-add agree; g >= 0 on the domain) holds at most one
// breakpoint, so with first[g] = #{i : cell(B_i) < g} = the count at the
// cell's smallest float, the count at x is first[g] + (x >= B[first[g] + 1]).
//
// V4: breakpoints T_1 .. T_15, domain |x| <= 12 without a clamp: the codes of
// a clamp to +-2.75 are those of the unclamped x (no threshold lies beyond),
// and |x / rms| <= sqrt(D) <= 11.32 for D <= 128 (rms >= |x_i| / sqrt(D), and
// the 1e-8 floor only lowers the ratio); NaN converts to cell 0, code 0.
// K3 (turbo_prod K, x clamped to +-2.5): the nibble (sign << 3 | code) and the
// level of the residual e = x - level form a step function over the 15
// breakpoints L_0 < T_1 < L_1 < ... < T_7 < L_7: past T_c the code is c,
// past L_c the sign is 1 (e >= 0 exactly when x >= L_c).  State
// m = #{breakpoints <= x} has code m >> 1, sign m & 1.
constexpr float kK3Off = 20.0f, kV4Off = 96.0f;
constexpr int kK3Cells = 41, kV4Cells = 193;
struct V4Row {
    float t;  // next threshold (+inf past the last)
    uint32_t code;
};
// K3 state m as three 8-byte rows, one array each (16 rows x 8 B = 128 B:
// every row of an array in its own pair of LDS banks, so random lookups by
// the lanes of a wave do not conflict).
struct K3RowA {
    float b, lo;  // next breakpoint (+inf past the last); level of state m
};
struct K3RowB {
    float hi;      // level of state m + 1
    uint32_t nlo;  // nibble of state m
};
struct K3RowC {
    uint32_t nhi, pad;  // nibble of state m + 1
};
struct alignas(16) PackTables {
    uint8_t v4_row[208];  // [g] = 8 * first[g] (byte offset of the V4 row), g < kV4Cells
    uint8_t k3_row[48];   // [g] = 8 * first[g] (byte offset in each K3 array), g < kK3Cells
    V4Row v4[16];
    K3RowA k3a[16];
    K3RowB k3b[16];
    K3RowC k3c[16];
};
namespace thr {
constexpr int cell(float x, float off) { return (int)(x * 8.0f + off); }
template <int N>
struct Points {
    float b[N + 1];  // b[1..N] sorted breakpoints
};
template <int N>
constexpr bool one_per_cell(const Points<N>& P, float off, int cells) {
    for (int i = 1; i <= N; ++i) {
        if (cell(P.b[i], off) < 0 || cell(P.b[i], off) >= cells) return false;
        if (i > 1 && !(cell(P.b[i], off) > cell(P.b[i - 1], off))) return false;
    }
    return true;
}
template <int N>
constexpr int first_in_cell(const Points<N>& P, float off, int g) {
    int n = 0;
    for (int i = 1; i <= N; ++i) n += cell(P.b[i], off) < g ? 1 : 0;
    return n;
}
constexpr Points<15> v4_points() {
    Points<15> p{};
    for (int i = 1; i < 16; ++i) p.b[i] = kV4T.t[i];
    return p;
}
constexpr Points<15> k3_points() {
    Points<15> p{};
    for (int i = 1; i <= 15; ++i) p.b[i] = (i & 1) ? kK3[(i - 1) / 2] : kK3T.t[i / 2];
    return p;
}
constexpr uint32_t k3_nibble(int m) { return (uint32_t)((m >> 1) | ((m & 1) << 3)); }
constexpr PackTables pack_tables() {
    PackTables p{};
    constexpr Points<15> v4p = v4_points(), k3p = k3_points();
    for (int g = 0; g < kV4Cells; ++g)
        p.v4_row[g] = (uint8_t)(sizeof(V4Row) * first_in_cell(v4p, kV4Off, g));
    for (int g = 0; g < kK3Cells; ++g)
        p.k3_row[g] = (uint8_t)(8 * first_in_cell(k3p, kK3Off, g));
    for (int l = 0; l < 16; ++l) p.v4[l] = {l < 15 ? v4p.b[l + 1] : __builtin_huge_valf(), (uint32_t)l};
    for (int m = 0; m < 16; ++m) {
        const int m1 = m < 15 ? m + 1 : m;
        p.k3a[m] = {m < 15 ? k3p.b[m + 1] : __builtin_huge_valf(), kK3[m >> 1]};
        p.k3b[m] = {kK3[m1 >> 1], k3_nibble(m)};
        p.k3c[m] = {k3_nibble(m1), 0u};
    }
    return p;
}
constexpr bool sorted(const Points<15>& P) {
    for (int i = 2; i <= 15; ++i)
        if (!(P.b[i] > P.b[i - 1])) return false;
    return true;
}
}  // namespace thr
static_assert(thr::sorted(thr::v4_points()) && thr::sorted(thr::k3_points()) &&
                  thr::one_per_cell(thr::v4_points(), kV4Off, kV4Cells) &&
                  thr::one_per_cell(thr::k3_points(), kK3Off, kK3Cells) &&
                  thr::cell(-2.5f, kK3Off) == 0 && thr::cell(2.5f, kK3Off) == kK3Cells - 1 &&
                  thr::cell(-12.0f, kV4Off) == 0 && thr::cell(12.0f, kV4Off) == kV4Cells - 1,
              "search grids");
static_assert(sizeof(V4Row) == 8 && sizeof(K3RowA) == 8 && sizeof(K3RowB) == 8 &&
                  sizeof(K3RowC) == 8 && sizeof(PackTables) % 16 == 0 &&
                  sizeof(PackTables) / 4 <= 256,
              "LDS table of whole dwords, rows aligned, one dword per thread of a block");
__device__ constexpr PackTables kPackTables = thr::pack_tables();
constexpr int kPackTableWords = sizeof(PackTables) / 4;

// Nearest V4 index of x (the reference's first-minimum scan of x clamped to
// +-2.75), for |x| <= 12 or NaN.
__device__ __forceinline__ uint32_t v4_code(float x, const PackTables& T) {
    const char* row =
        reinterpret_cast<const char*>(T.v4) + T.v4_row[(int)__builtin_fmaf(x, 8.0f, kV4Off)];
    const float t = *reinterpret_cast<const float*>(row);
    return *reinterpret_cast<const uint32_t*>(row + 4) + (x >= t ? 1u : 0u);
}
// turbo_prod K nibble (residual sign << 3 | nearest K3 index) of a clamped x,
// and the level of its residual.
__device__ __forceinline__ uint32_t k3_nibble(float x, const PackTables& T, float& level) {
    const uint32_t off = T.k3_row[(int)__builtin_fmaf(x, 8.0f, kK3Off)];
    const K3RowA a = *reinterpret_cast<const K3RowA*>(reinterpret_cast<const char*>(T.k3a) + off);
    const K3RowB b = *reinterpret_cast<const K3RowB*>(reinterpret_cast<const char*>(T.k3b) + off);
    const uint32_t nhi = reinterpret_cast<const K3RowC*>(reinterpret_cast<const char*>(T.k3c) + off)->nhi;
    const bool up = x >= a.b;
    level = up ? b.hi : a.lo;
    return up ? nhi : b.nlo;
}

// For the fp16 pair w = (a low, b high): d = fp32(a) - fp32(b) and
// s = fp32(a) + fp32(b), each rounded once, read straight from the halves
// (v_fma_mix_f32 computes a * 1.0 +- b in fp32 with one rounding; the fp16
// operands widen exactly).
__device__ __forceinline__ void half_pair_diff_sum(uint32_t w, float& d, float& s) {
    asm("v_fma_mix_f32 %0, %2, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[1,0,1]\n\t"
        "v_fma_mix_f32 %1, %2, 1.0, %2 op_sel:[0,0,1] op_sel_hi:[1,0,1]"
        : "=&v"(d), "=v"(s)
        : "v"(w));
}

// a / b rounded correctly, given y = RN(1/b) (Markstein's FMA division:
// q0 = RN(a * y) is within one ulp of a / b, the remainder a - b * q0 is then
// exact in one fma, and RN(q0 + remainder * y) is the correctly rounded
// quotient; P. Markstein, IBM J. Res. Dev. 34(1), 1990).  Valid while no
// step underflows or overflows: the pack divides rotated values by their
// row's RMS (>= 1e-8), quotients between 1e-14 and 1e14 or zero.
__device__ __forceinline__ float div_by(float a, float b, float y) {
    const float q0 = a * y;
    return fmaf(fmaf(-q0, b, a), y, q0);
}

// slot -> (page, token-in-block).
__device__ __forceinline__ void split_slot(int slot, const PageGeom& g, int& page, int& tib) {
    if (g.bs_shift >= 0) {
        page = slot >> g.bs_shift;
        tib = slot & ((1 << g.bs_shift) - 1);
    } else {
        page = slot / g.block_size;
        tib = slot % g.block_size;
    }
}

__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

// Non-temporal loads (data read once: the L2 keeps what is reused).
__device__ __forceinline__ uint16_t ld_u16_nt(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p));
}
__device__ __forceinline__ uint32_t ld_u32_nt(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}
__device__ __forceinline__ uint4 ld_u4_nt(const uint8_t* p) {
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    const v4u x = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(x[0], x[1], x[2], x[3]);
}

}  // namespace dev
}  // namespace tq

// Device code shared by the matrix-core kernels (affine_mfma.hip,
// affine_rows.hip): the code encoding, the activation staging that turns x
// into f16 hi/lo MFMA operands, and the per-tile product with its epilogue.
//
// Operand placement (v_mfma_f32_16x16x32_f16: A row i = lane%16, B column
// j = lane%16, both taking K chunk lane/16; D[i][j] lives in lane
// j + 16*(i/4), element i%4):
//   B operand = codes: lane (r, g) holds 8 codes of weight row r (one u32
//     word for Q4, two for Q8) from K chunk g.
//   A operand = activations: row i is a "slot" (quant group gamma, RHS t,
//     part hi/lo); it is non-zero only on the K chunks that belong to quant
//     group gamma, so one MFMA keeps the partial dots of different quant
//     groups in different D rows and each group's scale applies afterwards.
// A tile is 16 rows x 128 K; four MFMAs consume it. Lane (r, g) of D holds
// the four slots of one quant group and row r, so the epilogue is four FMAs
// for the scales and two for the biases.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qmr {
namespace mfma {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kTileK = 128;             // K per tile
constexpr uint32_t kOut = 0x80000000u;  // buffer offset past every range: loads return 0
constexpr uint32_t kRsrcWord3 = 0x00020000u;
constexpr int kAuxStream = 2;           // nt: streaming weights

template <int META>
__device__ __forceinline__ float meta_f32(uint32_t v) {
    if constexpr (META == 0) {
        return __uint_as_float(v);
    } else if constexpr (META == 1) {
        return __uint_as_float(v << 16);
    } else {
        return float(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v)));
    }
}

// Code encoding. A code is placed inside a 16-bit half so that the half is an
// IEEE f16 subnormal of value q * 2^-CODE_EXP. The matrix core rounds
// products of the smallest subnormals (codes in bits 0-3, q * 2^-24) with a
// biased error near 2^-22 of the dot product, while codes at bits 4-7 (Q4,
// q * 2^-20) or bits 2-9 (Q8, q * 2^-22) are as accurate as normal f16
// operands (about 2^-27 relative to the sum of |products|, unbiased); bits
// 10-14 are the exponent, so no higher placement is linear in q.
//   Q4 word -> halves [q0, q4 | q1, q5 | q2, q6 | q3, q7] * 2^-20
//   Q8 words w0,w1 -> [b0, b2 | b1, b3 | b4, b6 | b5, b7] * 2^-22
// k_of(e) is the column (within the 8-column chunk) of half e.
// BITS = 16: dense F16 weights, used as stored (no scale exponent, halves in
// column order).
template <int BITS>
constexpr int kCodeExp = BITS == 4 ? 20 : BITS == 8 ? 22 : 0;

template <int BITS>
__device__ __forceinline__ int k_of(int e) {
    if constexpr (BITS == 16) {
        return e;
    } else if constexpr (BITS == 4) {
        constexpr int k[8] = {0, 4, 1, 5, 2, 6, 3, 7};
        return k[e];
    } else {
        constexpr int k[8] = {0, 2, 1, 3, 4, 6, 5, 7};
        return k[e];
    }
}

template <int BITS>
__device__ __forceinline__ h8 unpack(const u4 (&c)[BITS / 4], int m) {
    u4 v;
    if constexpr (BITS == 4) {
        const uint32_t wd = c[0][m];
        v[0] = (wd << 4) & 0x00F000F0u;
        v[1] = wd & 0x00F000F0u;
        v[2] = (wd >> 4) & 0x00F000F0u;
        v[3] = (wd >> 8) & 0x00F000F0u;
    } else {
        const uint32_t w0 = c[(2 * m) >> 2][(2 * m) & 3];
        const uint32_t w1 = c[(2 * m + 1) >> 2][(2 * m + 1) & 3];
        v[0] = (w0 << 2) & 0x03FC03FCu;
        v[1] = (w0 >> 6) & 0x03FC03FCu;
        v[2] = (w1 << 2) & 0x03FC03FCu;
        v[3] = (w1 >> 6) & 0x03FC03FCu;
    }
    return __builtin_bit_cast(h8, v);
}

// Workgroup barrier ordering LDS only: outstanding global loads (the weight
// ring) stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// LDS written by some lanes of a wave and read by others of the same wave.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

template <int META>
__device__ __forceinline__ float meta_lo(uint32_t v) {  // entry packed as s | b << 16
    if constexpr (META == 1) return __uint_as_float(v << 16);
    return float(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v & 0xFFFFu)));
}
template <int META>
__device__ __forceinline__ float meta_hi(uint32_t v) {
    if constexpr (META == 1) return __uint_as_float(v & 0xFFFF0000u);
    return float(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v >> 16)));
}

// DPP lane exchange inside 16-lane rows. Every pattern used here reads a
// lane of the reader's own row, so with full row and bank masks no lane reads
// an invalid source and bound_ctrl changes nothing; it lets the compiler fold
// the exchange into the add or max that consumes it (v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <- 7 - i within 8 lanes
constexpr int kDppMirror = 0x140;     // lane i <- 15 - i within 16 lanes

// Sum and max over N (4, 8 or 16) consecutive, aligned lanes; every lane of
// the run receives both. After the quad steps a quad holds one value, so the
// mirrors pair each quad (then each half) with the other one. mx is a max of
// magnitudes: a non-negative float, whose bits order as unsigned integers,
// so its max runs on the bits (no NaN quieting between the steps).
template <int N>
__device__ __forceinline__ void group_reduce(float &sum, float &mx) {
    static_assert(N == 4 || N == 8 || N == 16, "runs of 4, 8 or 16 lanes");
    uint32_t m = __float_as_uint(mx);
    sum += dpp_f32<kDppXor1>(sum);
    m = max(m, dpp_u32<kDppXor1>(m));
    sum += dpp_f32<kDppXor2>(sum);
    m = max(m, dpp_u32<kDppXor2>(m));
    if constexpr (N >= 8) {
        sum += dpp_f32<kDppHalfMirror>(sum);
        m = max(m, dpp_u32<kDppHalfMirror>(m));
    }
    if constexpr (N >= 16) {
        sum += dpp_f32<kDppMirror>(sum);
        m = max(m, dpp_u32<kDppMirror>(m));
    }
    mx = __uint_as_float(m);
}

// f16 conversions with one rounding (v_fma_mix*_f16: the FP32 fma a*b + c,
// rounded to nearest even into one half of the result). The low-half forms
// start a fresh word; the high-half forms keep the word's low half.
//   hi_pair: (f16(a0*s), f16(a1*s))
//   lo_pair: (f16(a0*s - h.lo), f16(a1*s - h.hi)) for the f16 pair h
__device__ __forceinline__ uint32_t hi_pair(float a0, float a1, float s) {
    uint32_t d;
    asm("v_fma_mixlo_f16 %0, %1, %2, 0" : "=v"(d) : "v"(a0), "v"(s));
    asm("v_fma_mixhi_f16 %0, %1, %2, 0" : "+v"(d) : "v"(a1), "v"(s));
    return d;
}
__device__ __forceinline__ uint32_t lo_pair(float a0, float a1, float s, uint32_t h) {
    uint32_t d;
    asm("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel_hi:[0,0,1]" : "=v"(d) : "v"(a0), "v"(s), "v"(h));
    asm("v_fma_mixhi_f16 %0, %1, %2, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "+v"(d) : "v"(a1), "v"(s), "v"(h));
    return d;
}

// Staged activations of a run of K tiles, in LDS:
//   A   [tile][4 m][4 g][2B] u4: hi/lo f16 operand blocks of 8 columns
//   Sx  [tile][NGM][HALF/2] float4: (sum x_t, sum x_t+1, 2^(c+e_t), 2^(c+e_t+1))
// An x "item" is (tile Tl, RHS t, K chunk g, MFMA m): 8 consecutive columns
// at tile*128 + 32g + 8m. Items are numbered ((Tl*B + t)*4 + g)*4 + m, so
// the GROUP/8 items of one quant group sit in consecutive lanes.
struct ItemPos {
    uint32_t Tl;  // tile within the run
    int t, g, m;
};
template <int B>
__device__ __forceinline__ ItemPos item_pos(uint32_t it) {
    const uint32_t tt = it >> 4;
    return ItemPos{tt / B, int(tt % B), int((it >> 2) & 3), int(it & 3)};
}
// First column of an item, relative to the run's first column.
template <int B>
__device__ __forceinline__ uint32_t item_col(uint32_t it) {
    const ItemPos q = item_pos<B>(it);
    return q.Tl * kTileK + 32u * q.g + 8u * q.m;
}

// Loads the 8 columns of x[t] at column k (x view of B rows of cols floats);
// columns at or past cols, or a dead item, read as zeros. Two 128-bit loads
// whatever the view's alignment: multi-dword buffer loads need only 4-byte
// alignment, which every buffer offset has. (A runtime choice between load
// shapes here made the compiler wait for these loads before issuing the
// weight loads behind them.)
__device__ __forceinline__ void load_x8(float (&xv)[8], __amdgpu_buffer_rsrc_t xr, uint32_t t,
                                        uint32_t k, uint32_t cols, bool live) {
    const uint32_t xo = (live && k < cols) ? (t * cols + k) * 4u : kOut;
    const u4 a = __builtin_amdgcn_raw_buffer_load_b128(xr, int(xo), 0, 0);
    const u4 b = __builtin_amdgcn_raw_buffer_load_b128(xr, int(xo + 16u), 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        xv[j] = __uint_as_float(a[j]);
        xv[4 + j] = __uint_as_float(b[j]);
    }
}

// x as MFMA A operands: hi/lo f16 with a power-of-two scale per (quant
// group, RHS) taken from the group's max |x|, the group sums of x and the
// epilogue factors 2^(CODE_EXP + e). Every lane of the wave must call this
// (the group reductions shuffle across lanes); `store` says whether this
// lane's item exists.
template <int BITS, int GROUP, int B>
__device__ __forceinline__ void stage_x_item(const float (&xv)[8], uint32_t it, bool store, int lane,
                                             u4 *ldsA, float4 *ldsSx) {
    constexpr int NGM = kTileK / GROUP;
    constexpr int HALF = 16 / NGM / 2;
    const ItemPos q = item_pos<B>(it);
    // The item's sum (pairwise) and max |x|, then the group's.
    float psum = ((xv[0] + xv[1]) + (xv[2] + xv[3])) + ((xv[4] + xv[5]) + (xv[6] + xv[7]));
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(xv[j]));
    group_reduce<GROUP / 8>(psum, mx);
    const uint32_t mb = __float_as_uint(mx);
    int e = 0;
    if (mb != 0u && mb < 0x7F800000u) {
        e = int(mb >> 23) - 127 - 14;  // max * 2^-e in [2^14, 2^15) for normal max
        e = e < -100 ? -100 : (e > 100 ? 100 : e);
    }
    // x * 2^-e is exact (a power of two, within FP32's normal range), so hi is
    // its f16 rounding and lo the f16 rounding of the exact remainder.
    const float sc = __uint_as_float(uint32_t(127 - e) << 23);
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
        const float v0 = xv[k_of<BITS>(2 * e2)];
        const float v1 = xv[k_of<BITS>(2 * e2 + 1)];
        hw[e2] = hi_pair(v0, v1, sc);
        lw[e2] = lo_pair(v0, v1, sc, hw[e2]);
    }
    if (store) {
        u4 *dst = ldsA + ((q.Tl * 4 + q.m) * 4 + q.g) * (2 * B) + 2 * q.t;
        dst[0] = u4{hw[0], hw[1], hw[2], hw[3]};
        dst[1] = u4{lw[0], lw[1], lw[2], lw[3]};
        if ((lane & (GROUP / 8 - 1)) == 0) {
            float *s = reinterpret_cast<float *>(ldsSx + (q.Tl * NGM + (32 * q.g) / GROUP) * (HALF / 2) + q.t / 2);
            s[q.t & 1] = psum;
            s[2 + (q.t & 1)] = __uint_as_float(uint32_t(127 + kCodeExp<BITS> + e) << 23);
        }
    }
}

// Slots of absent RHS (B < HALF): zero sums and factors for `tiles` tiles.
template <int GROUP, int B>
__device__ __forceinline__ void stage_x_pads(uint32_t tiles, int tid, int nthr, float4 *ldsSx) {
    constexpr int NGM = kTileK / GROUP;
    constexpr int HALF = 16 / NGM / 2;
    if constexpr (HALF > B) {
        const uint32_t pads = tiles * NGM * (HALF - B);
        for (uint32_t it = tid; it < pads; it += nthr) {
            const uint32_t blk = it / (HALF - B);
            const uint32_t t = B + it % (HALF - B);
            float *s = reinterpret_cast<float *>(ldsSx + blk * (HALF / 2) + t / 2);
            s[t & 1] = 0.f;
            s[2 + (t & 1)] = 0.f;
        }
    }
}

// Per-lane constants of the A operand and the D epilogue.
//   A lane (slot i = r, chunk g = lg): non-zero when the slot's group is the
//   chunk's group and the slot's RHS exists; other lanes keep zeros.
//   D lane (row r, slots 4*lg .. 4*lg+3): group gD, RHS t0 (hi, lo), t0+1.
template <int GROUP, int B>
struct LaneMap {
    static constexpr int NGM = kTileK / GROUP;
    static constexpr int SLOTS = 16 / NGM;
    bool a_ok;
    uint32_t a_idx;
    int gD, t0;
    __device__ __forceinline__ explicit LaneMap(int lane) {
        const int r = lane & 15, lg = lane >> 4;
        const int a_slot = r % SLOTS;
        a_ok = (r / SLOTS) == (32 * lg) / GROUP && a_slot < 2 * B;
        a_idx = uint32_t(lg) * (2 * B) + uint32_t(a_ok ? a_slot : 0);
        gD = (4 * lg) / SLOTS;
        t0 = ((4 * lg) % SLOTS) / 2;
    }
};

// One 16-row x 128-column tile: unpack the codes, read this lane's A operand
// blocks, scale and bias (LDS metadata entry `mm`, staged sums sx) and four
// MFMAs into acc. a[] keeps zeros in lanes whose A operand is empty.
template <int BITS, int META, int GROUP, int B>
__device__ __forceinline__ void tile_product(const u4 (&c)[BITS / 4], const LaneMap<GROUP, B> &L,
                                             const u4 *ldsA_tile, float sv, float bv, float4 sx,
                                             h8 (&a)[4], float (&acc)[4]) {
    h8 bq[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) bq[m] = unpack<BITS>(c, m);
    if (L.a_ok) {
#pragma unroll
        for (int m = 0; m < 4; ++m) a[m] = __builtin_bit_cast(h8, ldsA_tile[m * (8 * B) + L.a_idx]);
    }
    f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m], bq[m], d, 0, 0, 0);
    const float s0 = sv * sx.z, s1 = sv * sx.w;
    acc[0] = __builtin_fmaf(s0, d[0], acc[0]);
    acc[1] = __builtin_fmaf(s0, d[1], acc[1]);
    acc[2] = __builtin_fmaf(s1, d[2], acc[2]);
    acc[3] = __builtin_fmaf(s1, d[3], acc[3]);
    acc[0] = __builtin_fmaf(bv, sx.x, acc[0]);
    acc[2] = __builtin_fmaf(bv, sx.y, acc[2]);
}

// Metadata entry of LDS word(s) at `m` (packed s | b << 16, or two F32 words).
template <int META>
__device__ __forceinline__ void meta_entry(const uint32_t *m, float &sv, float &bv) {
    if constexpr (META == 0) {
        const uint2 mm = *reinterpret_cast<const uint2 *>(m);
        sv = __uint_as_float(mm.x);
        bv = __uint_as_float(mm.y);
    } else {
        const uint32_t mm = *m;
        sv = meta_lo<META>(mm);
        bv = meta_hi<META>(mm);
    }
}

// Combines a lane's hi/lo slots and the quant groups of D: afterwards lanes
// with lg < 4/NGM hold the row's sums for RHS t0 (v0) and t0 + 1 (v1).
template <int GROUP>
__device__ __forceinline__ void combine_slots(const float (&acc)[4], float &v0, float &v1) {
    constexpr int NGM = kTileK / GROUP;
    v0 = acc[0] + acc[1];
    v1 = acc[2] + acc[3];
    if constexpr (NGM == 4) {
        v0 += __shfl_xor(v0, 16);
        v1 += __shfl_xor(v1, 16);
    }
    if constexpr (NGM >= 2) {
        v0 += __shfl_xor(v0, 32);
        v1 += __shfl_xor(v1, 32);
    }
}

}  // namespace mfma
}  // namespace qmr

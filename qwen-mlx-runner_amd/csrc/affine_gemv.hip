// Fused dequantise + GEMV / small block (batch 1..4) over MLX affine packed
// weights, hand-written for gfx950 (CDNA4, wave64).
//
// Computes, for every RHS t and output row r,
//     y[t*rows + r] = sum_c (q[r,c] * s[r,g(c)] + b[r,g(c)]) * x[t*cols + c]
// which is the arithmetic of the reference's affine() / matvec_affine
// (kernels/qwen.metal:40-68) and its block form (kernels/matmul_block.metal).
//
// Layout in HBM (unchanged from the checkpoint, src/weights.rs:322-326):
//   w : u32 [rows][cols*bits/32]; field c of a row sits at bits (c%pack)*bits
//       of word c/pack, little-endian.
//   s, b : [rows][cols/group] as FP32, BF16 (high half of FP32) or F16.
//   x : FP32 [batch][cols]; y : FP32 [batch][rows].
//
// Work decomposition. A "chunk" is 16 bytes of one row: 32 Q4 codes or 16 Q8
// codes, always inside one quantisation group (group >= 32). A half-wave (32
// lanes) is a row slot: in one round it reads 32 consecutive chunks of a row
// (512 contiguous bytes, one 128-bit load per lane) for each of its RR rows.
// A 256-thread workgroup has 8 slots; KS slots share a row group and split its
// rounds (t = kp, kp+KS, ...), their partial sums meeting in LDS. The
// activation vectors are staged once per workgroup in LDS together with each
// chunk's sum of x; each lane reads its chunk's x from LDS once per round and
// reuses it for all RR rows.
//
// Unpack. Masking a word with 0x000F000F leaves two IEEE half subnormals whose
// values are exactly q*2^-24 (q = nibble 0 and nibble 4); 0x00F000F0 leaves
// q*2^-20 (nibbles 1 and 5); the word shifted by 8 gives nibbles 2,6 and 3,7
// the same way. v_fma_mix_f32 consumes a half operand directly, so every
// weight costs one mask share (5 ops per 8 codes) and one fused multiply-add,
// with no integer-to-float conversion. Products are exact and accumulate in
// FP32; the 2^24 / 2^20 factors are restored once per chunk:
//     qdot = 2^24 * (acc_even + acc_odd / 16)
// and the affine form is applied per chunk as s*qdot + b*sum(x_chunk)
// (the factorisation of kernels/matvec_fast.metal:11-15). Q8 uses
// 0x00FF00FF masks (byte values up to 255 are half subnormals too).
// The kernel descriptor keeps f16 denormals (float_denorm_mode_16_64 = 3),
// which this unpack relies on.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.hpp"

namespace qmr {
namespace {

constexpr int kThreads = 256;
constexpr int kSlots = kThreads / 32;  // half-wave row slots per workgroup

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }

template <int META>
__device__ __forceinline__ float load_meta(const void *p, size_t i) {
    if constexpr (META == 0) {
        return static_cast<const float *>(p)[i];
    } else if constexpr (META == 1) {
        return __uint_as_float(uint32_t(static_cast<const uint16_t *>(p)[i]) << 16);
    } else {
        return float(__builtin_bit_cast(_Float16, static_cast<const uint16_t *>(p)[i]));
    }
}

// DPP / swizzle butterfly over each 32-lane half of the wave. Every lane ends
// with its half-wave's total; the order of additions is fixed.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float half_wave_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
    v += dpp<0x141>(v);  // row_half_mirror: the other quad of each 8
    v += dpp<0x140>(v);  // row_mirror: the other 8 of each 16
    // ds_swizzle bit mode, and_mask 0x1f, xor_mask 0x10: the other 16 of 32.
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
    return v;
}

// Units of 16 bytes per chunk in the staged x: 8 (Q4, 32 floats), 4 (Q8).
template <int BITS>
struct Geo {
    static constexpr int kChunkCols = 128 / BITS;  // columns per 16-byte chunk
    static constexpr int kUnits = kChunkCols / 4;  // float4 units of x per chunk
    static constexpr int kUnitShift = BITS == 4 ? 3 : 2;
};

// XOR swizzle of float4 units inside each chunk so that the 32 lanes of a
// slot, which read chunk-strided addresses, spread over the LDS banks.
template <int BITS>
__device__ __forceinline__ uint32_t swz(uint32_t unit) {
    constexpr uint32_t m = Geo<BITS>::kUnits - 1;
    return unit ^ ((unit >> Geo<BITS>::kUnitShift) & m);
}

// Dot of one Q4 chunk (4 words, 32 codes) with its 32 x values.
__device__ __forceinline__ void q4_chunk(const uint32_t (&d)[4], const float4 (&xv)[8], float &ae,
                                         float &ao) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t a = d[j] & 0x000F000Fu;
        const uint32_t b = d[j] & 0x00F000F0u;
        const uint32_t d8 = d[j] >> 8;
        const uint32_t c = d8 & 0x000F000Fu;
        const uint32_t e = d8 & 0x00F000F0u;
        const half2v ha = as_h2(a), hb = as_h2(b), hc = as_h2(c), he = as_h2(e);
        const float4 lo = xv[2 * j], hi = xv[2 * j + 1];
        ae = __builtin_fmaf(float(ha.x), lo.x, ae);
        ao = __builtin_fmaf(float(hb.x), lo.y, ao);
        ae = __builtin_fmaf(float(hc.x), lo.z, ae);
        ao = __builtin_fmaf(float(he.x), lo.w, ao);
        ae = __builtin_fmaf(float(ha.y), hi.x, ae);
        ao = __builtin_fmaf(float(hb.y), hi.y, ao);
        ae = __builtin_fmaf(float(hc.y), hi.z, ae);
        ao = __builtin_fmaf(float(he.y), hi.w, ao);
    }
}

// Dot of one Q8 chunk (4 words, 16 codes) with its 16 x values.
__device__ __forceinline__ void q8_chunk(const uint32_t (&d)[4], const float4 (&xv)[4], float &ae,
                                         float &ao) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t lo = d[j] & 0x00FF00FFu;
        const uint32_t hi = (d[j] >> 8) & 0x00FF00FFu;
        const half2v hl = as_h2(lo), hh = as_h2(hi);
        const float4 xx = xv[j];
        ae = __builtin_fmaf(float(hl.x), xx.x, ae);
        ao = __builtin_fmaf(float(hh.x), xx.y, ao);
        ae = __builtin_fmaf(float(hl.y), xx.z, ae);
        ao = __builtin_fmaf(float(hh.y), xx.w, ao);
    }
}

template <int RR>
struct Stage {
    uint32_t w[RR][4];
    float s[RR], b[RR];
};

template <int BITS, int META, int B, int RR, int KS, bool XLDS>
__global__ __launch_bounds__(kThreads) void affine_gemv_kernel(
    const uint32_t *__restrict__ w, const void *__restrict__ sp, const void *__restrict__ bp,
    const float *__restrict__ x, float *__restrict__ y, uint32_t rows, uint32_t cols,
    uint32_t group_shift, uint32_t vec16) {
    using G = Geo<BITS>;
    constexpr int kUnits = G::kUnits;
    constexpr int kRowGroups = kSlots / KS;
    constexpr int kRowsPerWg = kRowGroups * RR;

    extern __shared__ float4 lds4[];
    const uint32_t C = cols / G::kChunkCols;  // chunks per row
    const uint32_t rounds = (C + 31) / 32;
    const uint32_t units = cols / 4;          // float4 units per x vector
    float4 *xs = lds4;                        // [B][units] swizzled (XLDS)
    float *xsum = reinterpret_cast<float *>(lds4 + (XLDS ? B * units : 0));  // [B][C]
    float *part = xsum + B * C;               // [KS][kRowsPerWg][B]

    const int tid = threadIdx.x;
    const int lane = tid & 31;
    const int slot = tid >> 5;
    const int rg = slot / KS;
    const int kp = slot % KS;

    // Stage x (and per-chunk sums) into LDS. Scalar loads: x views need only
    // 4-byte alignment. Each chunk is summed by one thread in column order.
    for (uint32_t ck = tid; ck < B * C; ck += kThreads) {
        const uint32_t t = ck / C, chunk = ck % C;
        const float *src = x + size_t(t) * cols + size_t(chunk) * G::kChunkCols;
        float sum = 0.f;
#pragma unroll
        for (int u = 0; u < kUnits; ++u) {
            float4 v = make_float4(src[4 * u], src[4 * u + 1], src[4 * u + 2], src[4 * u + 3]);
            sum += v.x;
            sum += v.y;
            sum += v.z;
            sum += v.w;
            if constexpr (XLDS) xs[t * units + swz<BITS>(chunk * kUnits + u)] = v;
        }
        xsum[ck] = sum;
    }
    __syncthreads();

    const uint32_t row0 = blockIdx.x * kRowsPerWg + rg * RR;
    const uint32_t groups = cols >> group_shift;
    float acc[RR][B];
#pragma unroll
    for (int i = 0; i < RR; ++i)
#pragma unroll
        for (int t = 0; t < B; ++t) acc[i][t] = 0.f;

    auto load_stage = [&](uint32_t round, Stage<RR> &st) {
        const uint32_t chunk = round * 32 + lane;
        const bool cv = chunk < C;
        const uint32_t gi_col = (chunk * G::kChunkCols) >> group_shift;
#pragma unroll
        for (int i = 0; i < RR; ++i) {
            const uint32_t row = row0 + i;
            if (cv && row < rows) {
                const uint32_t *src = w + (size_t(row) * C + chunk) * 4;
                if (vec16) {
                    const uint4 v = *reinterpret_cast<const uint4 *>(src);
                    st.w[i][0] = v.x;
                    st.w[i][1] = v.y;
                    st.w[i][2] = v.z;
                    st.w[i][3] = v.w;
                } else {
                    st.w[i][0] = src[0];
                    st.w[i][1] = src[1];
                    st.w[i][2] = src[2];
                    st.w[i][3] = src[3];
                }
                const size_t gi = size_t(row) * groups + gi_col;
                st.s[i] = load_meta<META>(sp, gi);
                st.b[i] = load_meta<META>(bp, gi);
            } else {
                st.w[i][0] = st.w[i][1] = st.w[i][2] = st.w[i][3] = 0u;
                st.s[i] = 0.f;
                st.b[i] = 0.f;
            }
        }
    };

    auto compute = [&](uint32_t round, const Stage<RR> &st) {
        const uint32_t chunk = round * 32 + lane;
        if (chunk >= C) return;
        float4 xv[B][kUnits];
        float xsv[B];
#pragma unroll
        for (int t = 0; t < B; ++t) {
            if constexpr (XLDS) {
#pragma unroll
                for (int u = 0; u < kUnits; ++u) xv[t][u] = xs[t * units + swz<BITS>(chunk * kUnits + u)];
                xsv[t] = xsum[t * C + chunk];
            } else {
                const float *src = x + size_t(t) * cols + size_t(chunk) * G::kChunkCols;
#pragma unroll
                for (int u = 0; u < kUnits; ++u)
                    xv[t][u] = make_float4(src[4 * u], src[4 * u + 1], src[4 * u + 2], src[4 * u + 3]);
                xsv[t] = xsum[t * C + chunk];
            }
        }
#pragma unroll
        for (int i = 0; i < RR; ++i) {
            if (row0 + i >= rows) continue;
            const float s24 = st.s[i] * 16777216.0f;  // 2^24, exact
#pragma unroll
            for (int t = 0; t < B; ++t) {
                float ae = 0.f, ao = 0.f, q;
                if constexpr (BITS == 4) {
                    q4_chunk(st.w[i], xv[t], ae, ao);
                    q = __builtin_fmaf(ao, 0.0625f, ae);
                } else {
                    q8_chunk(st.w[i], xv[t], ae, ao);
                    q = ae + ao;
                }
                acc[i][t] = __builtin_fmaf(s24, q, acc[i][t]);
                acc[i][t] = __builtin_fmaf(st.b[i], xsv[t], acc[i][t]);
            }
        }
    };

    // Software pipeline: the next round's loads are in flight while the
    // current round computes (ping-pong register stages, no copies).
    if (uint32_t(kp) < rounds) {
        Stage<RR> sa, sb;
        uint32_t t = kp;
        load_stage(t, sa);
        while (true) {
            uint32_t tn = t + KS;
            if (tn < rounds) load_stage(tn, sb);
            compute(t, sa);
            t = tn;
            if (t >= rounds) break;
            tn = t + KS;
            if (tn < rounds) load_stage(tn, sa);
            compute(t, sb);
            t = tn;
            if (t >= rounds) break;
        }
    }

    // Reduce each row's lane partials across the slot, then across the KS
    // slots of the row group (fixed order), and store.
#pragma unroll
    for (int i = 0; i < RR; ++i) {
#pragma unroll
        for (int t = 0; t < B; ++t) {
            const float v = half_wave_sum(acc[i][t]);
            const uint32_t row = row0 + i;
            if (lane == 0) {
                if constexpr (KS == 1) {
                    if (row < rows) y[size_t(t) * rows + row] = v;
                } else {
                    part[(kp * kRowsPerWg + rg * RR + i) * B + t] = v;
                }
            }
        }
    }
    if constexpr (KS > 1) {
        __syncthreads();
        for (int idx = tid; idx < kRowsPerWg * B; idx += kThreads) {
            const int rl = idx / B, t = idx % B;
            const uint32_t row = blockIdx.x * kRowsPerWg + rl;
            if (row < rows) {
                float v = part[rl * B + t];
#pragma unroll
                for (int k = 1; k < KS; ++k) v += part[(k * kRowsPerWg + rl) * B + t];
                y[size_t(t) * rows + row] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Streaming variant: one 16-wave workgroup per CU (32 half-wave slots).
//
// A workgroup owns R consecutive rows and all T rounds of them. Its T*R
// (round, row) units are numbered round-major and dealt to the 32 slots in
// contiguous, equal runs (R*T/32 units each, +-1), so every slot streams the
// same number of bytes and mostly walks down rows at one fixed round: the x
// chunk it reads from LDS is reused across its whole run. Each slot keeps P
// units of loads in flight in a register ring (weights, scale, bias), issued
// before x is staged, so the workgroup's first HBM requests leave at once
// and the ring then refills one unit behind each unit consumed. A unit's
// lane partials are reduced across the slot (DPP + swizzle) and parked in
// LDS at [round][row]; after a barrier every row is summed over its rounds in
// round order, so the result is deterministic.
// ---------------------------------------------------------------------------
constexpr int kUThreads = 1024;
constexpr int kUSlots = kUThreads / 32;

template <int B>
struct Ring {
    uint32_t w[4];
    float s, b;
};

template <int BITS, int META, int B, int P, bool XLDS>
__global__ __launch_bounds__(kUThreads) void affine_gemv_units_kernel(
    const uint32_t *__restrict__ w, const void *__restrict__ sp, const void *__restrict__ bp,
    const float *__restrict__ x, float *__restrict__ y, uint32_t rows, uint32_t cols,
    uint32_t group_shift, uint32_t vec16, uint32_t rows_per_wg) {
    using G = Geo<BITS>;
    constexpr int kUnits = G::kUnits;
    extern __shared__ float4 lds4[];
    const uint32_t C = cols / G::kChunkCols;
    const uint32_t T = (C + 31) / 32;
    const uint32_t units4 = cols / 4;
    const uint32_t r0 = blockIdx.x * rows_per_wg;
    const uint32_t R = rows - r0 < rows_per_wg ? rows - r0 : rows_per_wg;
    float4 *xs = lds4;
    float *xsum = reinterpret_cast<float *>(lds4 + (XLDS ? B * units4 : 0));  // [B][C]
    float *part = xsum + B * C;                                                // [B][T][rows_per_wg]

    const int tid = threadIdx.x;
    const int lane = tid & 31;
    const int slot = tid >> 5;
    const uint32_t n_units = T * R;
    const uint32_t u_begin = uint32_t(uint64_t(n_units) * slot / kUSlots);
    const uint32_t u_end = uint32_t(uint64_t(n_units) * (slot + 1) / kUSlots);
    const uint32_t groups = cols >> group_shift;

    // Issue cursor (it, ir) and compute cursor (ct, cr) over round-major units.
    uint32_t it = u_begin / R, ir = u_begin % R;
    uint32_t ct = it, cr = ir;

    Ring<B> ring[P];
    auto issue = [&](Ring<B> &sl, bool active) {
        const uint32_t chunk = it * 32 + lane;
        const uint32_t row = r0 + ir;
        if (active && chunk < C) {
            const uint32_t *src = w + (size_t(row) * C + chunk) * 4;
            if (vec16) {
                const uint4 v = *reinterpret_cast<const uint4 *>(src);
                sl.w[0] = v.x;
                sl.w[1] = v.y;
                sl.w[2] = v.z;
                sl.w[3] = v.w;
            } else {
                sl.w[0] = src[0];
                sl.w[1] = src[1];
                sl.w[2] = src[2];
                sl.w[3] = src[3];
            }
            const size_t gi = size_t(row) * groups + ((chunk * G::kChunkCols) >> group_shift);
            sl.s = load_meta<META>(sp, gi);
            sl.b = load_meta<META>(bp, gi);
        } else {
            sl.w[0] = sl.w[1] = sl.w[2] = sl.w[3] = 0u;
            sl.s = 0.f;
            sl.b = 0.f;
        }
        if (++ir == R) {
            ir = 0;
            ++it;
        }
    };

#pragma unroll
    for (int j = 0; j < P; ++j) issue(ring[j], u_begin + j < u_end);

    // Stage x and per-chunk sums while the first weight loads are in flight.
    for (uint32_t ck = tid; ck < B * C; ck += kUThreads) {
        const uint32_t t = ck / C, chunk = ck % C;
        const float *src = x + size_t(t) * cols + size_t(chunk) * G::kChunkCols;
        float sum = 0.f;
#pragma unroll
        for (int u = 0; u < kUnits; ++u) {
            const float4 v = make_float4(src[4 * u], src[4 * u + 1], src[4 * u + 2], src[4 * u + 3]);
            sum += v.x;
            sum += v.y;
            sum += v.z;
            sum += v.w;
            if constexpr (XLDS) xs[t * units4 + swz<BITS>(chunk * kUnits + u)] = v;
        }
        xsum[ck] = sum;
    }
    __syncthreads();

    float4 xv[B][kUnits];
    float xsv[B];
    uint32_t cur_t = 0xFFFFFFFFu;
    for (uint32_t base = u_begin; base < u_end; base += P) {
#pragma unroll
        for (int j = 0; j < P; ++j) {
            const uint32_t u = base + j;
            if (u < u_end) {
                const uint32_t chunk = ct * 32 + lane;
                const bool cv = chunk < C;
                if (ct != cur_t) {
                    cur_t = ct;
#pragma unroll
                    for (int t = 0; t < B; ++t) {
                        if (cv) {
                            if constexpr (XLDS) {
#pragma unroll
                                for (int k = 0; k < kUnits; ++k)
                                    xv[t][k] = xs[t * units4 + swz<BITS>(chunk * kUnits + k)];
                            } else {
                                const float *src = x + size_t(t) * cols + size_t(chunk) * G::kChunkCols;
#pragma unroll
                                for (int k = 0; k < kUnits; ++k)
                                    xv[t][k] = make_float4(src[4 * k], src[4 * k + 1], src[4 * k + 2],
                                                           src[4 * k + 3]);
                            }
                            xsv[t] = xsum[t * C + chunk];
                        } else {
#pragma unroll
                            for (int k = 0; k < kUnits; ++k) xv[t][k] = make_float4(0.f, 0.f, 0.f, 0.f);
                            xsv[t] = 0.f;
                        }
                    }
                }
                const Ring<B> &sl = ring[j];
                const float s24 = sl.s * 16777216.0f;  // 2^24, exact
#pragma unroll
                for (int t = 0; t < B; ++t) {
                    float ae = 0.f, ao = 0.f, q;
                    if constexpr (BITS == 4) {
                        q4_chunk(sl.w, xv[t], ae, ao);
                        q = __builtin_fmaf(ao, 0.0625f, ae);
                    } else {
                        q8_chunk(sl.w, xv[t], ae, ao);
                        q = ae + ao;
                    }
                    float p = __builtin_fmaf(sl.b, xsv[t], s24 * q);
                    p = half_wave_sum(p);
                    if (lane == 0) part[(t * T + ct) * rows_per_wg + cr] = p;
                }
                if (++cr == R) {
                    cr = 0;
                    ++ct;
                }
            }
            if (u + P < u_end) issue(ring[j], true);
        }
    }
    __syncthreads();
    for (uint32_t idx = tid; idx < R * B; idx += kUThreads) {
        const uint32_t t = idx / R, r = idx % R;
        const float *pp = part + size_t(t) * T * rows_per_wg + r;
        float v = pp[0];
        for (uint32_t k = 1; k < T; ++k) v += pp[size_t(k) * rows_per_wg];
        y[size_t(t) * rows + r0 + r] = v;
    }
}

template <int BITS, int META, int B, int P, bool XLDS>
hipError_t launch_units(const AffineArgs &a, hipStream_t stream, size_t lds_bytes, uint32_t group_shift,
                        uint32_t vec16, uint32_t rows_per_wg) {
    auto kernel = affine_gemv_units_kernel<BITS, META, B, P, XLDS>;
    if (lds_bytes > 65536) {
        const hipError_t e = raise_lds_limit(reinterpret_cast<const void *>(kernel), lds_bytes);
        if (e != hipSuccess) return e;
    }
    const uint32_t blocks = (a.rows + rows_per_wg - 1) / rows_per_wg;
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kUThreads), lds_bytes, stream, a.w, a.s, a.b, a.x,
                       a.y, a.rows, a.cols, group_shift, vec16, rows_per_wg);
    return hipGetLastError();
}

template <int BITS, int META, int B, bool XLDS>
hipError_t units_meta(const AffineArgs &a, hipStream_t stream, size_t lds, uint32_t gs,
                      uint32_t vec16, uint32_t rpw) {
    return launch_units<BITS, META, B, 8, XLDS>(a, stream, lds, gs, vec16, rpw);
}

template <int BITS, int META, int B, int RR, int KS, bool XLDS>
hipError_t launch_instance(const AffineArgs &a, hipStream_t stream, size_t lds_bytes,
                           uint32_t group_shift, uint32_t vec16) {
    auto kernel = affine_gemv_kernel<BITS, META, B, RR, KS, XLDS>;
    if (lds_bytes > 65536) {
        const hipError_t e = raise_lds_limit(reinterpret_cast<const void *>(kernel), lds_bytes);
        if (e != hipSuccess) return e;
    }
    constexpr int kRowsPerWg = (kSlots / KS) * RR;
    const uint32_t blocks = (a.rows + kRowsPerWg - 1) / kRowsPerWg;
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kThreads), lds_bytes, stream, a.w, a.s, a.b, a.x,
                       a.y, a.rows, a.cols, group_shift, vec16);
    return hipGetLastError();
}

// (rr, ks) pairs compiled for every (bits, meta, batch).
constexpr int kPlans[][2] = {{1, 1}, {2, 1}, {4, 1}, {5, 2}, {2, 2}};

template <int BITS, int META, int B, bool XLDS>
hipError_t dispatch_plan(const AffineArgs &a, GemvPlan p, hipStream_t stream, size_t lds,
                         uint32_t gs, uint32_t vec16) {
    if (p.rr == 1 && p.ks == 1) return launch_instance<BITS, META, B, 1, 1, XLDS>(a, stream, lds, gs, vec16);
    if (p.rr == 2 && p.ks == 1) return launch_instance<BITS, META, B, 2, 1, XLDS>(a, stream, lds, gs, vec16);
    if (p.rr == 4 && p.ks == 1) return launch_instance<BITS, META, B, 4, 1, XLDS>(a, stream, lds, gs, vec16);
    if (p.rr == 5 && p.ks == 2) return launch_instance<BITS, META, B, 5, 2, XLDS>(a, stream, lds, gs, vec16);
    if (p.rr == 2 && p.ks == 2) return launch_instance<BITS, META, B, 2, 2, XLDS>(a, stream, lds, gs, vec16);
    return hipErrorInvalidValue;
}

template <int BITS, int META, int B>
hipError_t dispatch_x(const AffineArgs &a, GemvPlan p, hipStream_t stream, bool xlds, size_t lds,
                      uint32_t gs, uint32_t vec16) {
    return xlds ? dispatch_plan<BITS, META, B, true>(a, p, stream, lds, gs, vec16)
                : dispatch_plan<BITS, META, B, false>(a, p, stream, lds, gs, vec16);
}

template <int BITS, int META>
hipError_t dispatch_b(const AffineArgs &a, GemvPlan p, hipStream_t stream, bool xlds, size_t lds,
                      uint32_t gs, uint32_t vec16) {
    switch (a.batch) {
        case 1: return dispatch_x<BITS, META, 1>(a, p, stream, xlds, lds, gs, vec16);
        case 2: return dispatch_x<BITS, META, 2>(a, p, stream, xlds, lds, gs, vec16);
        case 3: return dispatch_x<BITS, META, 3>(a, p, stream, xlds, lds, gs, vec16);
        case 4: return dispatch_x<BITS, META, 4>(a, p, stream, xlds, lds, gs, vec16);
        default: return hipErrorInvalidValue;
    }
}

size_t lds_bytes_for(const AffineArgs &a, GemvPlan p, bool xlds) {
    const size_t chunk_cols = 128 / a.bits;
    const size_t C = a.cols / chunk_cols;
    const size_t rows_per_wg = size_t(kSlots / p.ks) * p.rr;
    size_t bytes = size_t(a.batch) * C * 4;  // chunk sums
    if (xlds) bytes += size_t(a.batch) * a.cols * 4;
    if (p.ks > 1) bytes += size_t(p.ks) * rows_per_wg * a.batch * 4;
    return bytes;
}

}  // namespace

GemvPlan plan_affine_gemv(const AffineArgs &a, GemvPlan forced, const DeviceLimits &lim) {
    if (forced.rr == -1) return {-1, 0};
    if (forced.rr > 0 && forced.ks > 0) {
        for (auto &pp : kPlans)
            if (pp[0] == forced.rr && pp[1] == forced.ks) return forced;
    }
    // Single-RHS products stream through CU-sized workgroups (rr = -1).
    if (a.batch == 1) return {-1, 0};
    // Blocks keep the row-slot kernel: long rows with few of them per CU
    // split K across two slots so that a workgroup of 20 rows covers one CU;
    // tall matrices keep whole rows per slot.
    const uint32_t chunk_cols = 128 / a.bits;
    const uint32_t rounds = (a.cols / chunk_cols + 31) / 32;
    const double rows_per_cu = double(a.rows) / double(lim.num_cus > 0 ? lim.num_cus : 256);
    GemvPlan p;
    if (rows_per_cu >= 256) {
        p = {4, 1};
    } else if (rows_per_cu >= 48) {
        p = {2, 1};
    } else if (rounds >= 4 && rows_per_cu >= 10) {
        p = {5, 2};
    } else if (rounds >= 2 && rows_per_cu >= 4) {
        p = {2, 2};
    } else {
        p = {1, 1};
    }
    return p;
}

namespace {

template <int BITS, int META>
hipError_t units_b(const AffineArgs &a, hipStream_t stream, bool xlds, size_t lds, uint32_t gs,
                   uint32_t vec16, uint32_t rpw) {
    if (a.batch != 1) return hipErrorInvalidValue;
    return xlds ? units_meta<BITS, META, 1, true>(a, stream, lds, gs, vec16, rpw)
                : units_meta<BITS, META, 1, false>(a, stream, lds, gs, vec16, rpw);
}

hipError_t launch_units_kernel(const AffineArgs &a, const DeviceLimits &lim, hipStream_t stream,
                               uint32_t gs, uint32_t vec16) {
    const uint32_t cus = lim.num_cus > 0 ? uint32_t(lim.num_cus) : 256u;
    const uint32_t grid = a.rows < cus ? a.rows : cus;
    const uint32_t rpw = (a.rows + grid - 1) / grid;
    const size_t C = a.cols / (128 / a.bits);
    const size_t T = (C + 31) / 32;
    size_t lds = size_t(a.batch) * (C + T * rpw) * 4;
    bool xlds = true;
    if (lds + size_t(a.batch) * a.cols * 4 <= lim.max_lds_per_block) {
        lds += size_t(a.batch) * a.cols * 4;
    } else {
        xlds = false;
        if (lds > lim.max_lds_per_block) return hipErrorInvalidValue;
    }
    const int meta = static_cast<int>(a.meta);
    if (a.bits == 4) {
        if (meta == 0) return units_b<4, 0>(a, stream, xlds, lds, gs, vec16, rpw);
        if (meta == 1) return units_b<4, 1>(a, stream, xlds, lds, gs, vec16, rpw);
        return units_b<4, 2>(a, stream, xlds, lds, gs, vec16, rpw);
    }
    if (meta == 0) return units_b<8, 0>(a, stream, xlds, lds, gs, vec16, rpw);
    if (meta == 1) return units_b<8, 1>(a, stream, xlds, lds, gs, vec16, rpw);
    return units_b<8, 2>(a, stream, xlds, lds, gs, vec16, rpw);
}

}  // namespace

hipError_t launch_affine_gemv(const AffineArgs &a, GemvPlan forced, const DeviceLimits &lim,
                              hipStream_t stream) {
    GemvPlan p = plan_affine_gemv(a, forced, lim);
    uint32_t gs = 0;
    while ((1u << gs) < a.group) ++gs;
    if ((1u << gs) != a.group) return hipErrorInvalidValue;
    const uint32_t vec16 = (reinterpret_cast<uintptr_t>(a.w) & 15) == 0 ? 1u : 0u;
    if (p.rr == -1) {
        if (a.batch == 1) return launch_units_kernel(a, lim, stream, gs, vec16);
        p = plan_affine_gemv(a, GemvPlan{}, lim);  // blocks use the row-slot kernel
        if (p.rr == -1) p = {1, 1};
    }
    bool xlds = true;
    size_t lds = lds_bytes_for(a, p, true);
    if (lds > lim.max_lds_per_block) {
        xlds = false;
        lds = lds_bytes_for(a, p, false);
        if (lds > lim.max_lds_per_block) return hipErrorInvalidValue;
    }
    const int meta = static_cast<int>(a.meta);
    if (a.bits == 4) {
        if (meta == 0) return dispatch_b<4, 0>(a, p, stream, xlds, lds, gs, vec16);
        if (meta == 1) return dispatch_b<4, 1>(a, p, stream, xlds, lds, gs, vec16);
        return dispatch_b<4, 2>(a, p, stream, xlds, lds, gs, vec16);
    }
    if (meta == 0) return dispatch_b<8, 0>(a, p, stream, xlds, lds, gs, vec16);
    if (meta == 1) return dispatch_b<8, 1>(a, p, stream, xlds, lds, gs, vec16);
    return dispatch_b<8, 2>(a, p, stream, xlds, lds, gs, vec16);
}

}  // namespace qmr

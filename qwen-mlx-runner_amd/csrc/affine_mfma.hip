// Streaming dequantise + GEMV / small block (batch 1..4) over MLX affine
// packed weights on the gfx950 matrix cores.
//
// Computes, for every RHS t < B and output row r,
//     y[t*rows + r] = sum_g ( s[r,g] * sum_{c in g} q[r,c] * x[t,c]
//                           + b[r,g] * sum_{c in g} x[t,c] )
// which is the reference's per-weight affine dot (kernels/qwen.metal:40-68,
// kernels/matmul_block.metal:20-79) in the factored form of
// kernels/matvec_fast.metal:11-15.
//
// Why MFMA for a memory-bound product. Dequantising on the vector ALU costs
// one FMA per weight per RHS plus the unpack (about 1.6 lane-ops per weight
// at B=1 and 4.6 at B=3), while HBM delivers Q4/g64 at about 1.4e13 weights/s
// against 3.9e13 VALU lane-ops/s: B=3 would be ALU-bound. Here the unpack is
// the only per-weight ALU work (7 ops per 8 codes, for any B up to 4); the
// products run on v_mfma_f32_16x16x32_f16, which has more than 10x headroom.
//
// Exactness. A Q4 code shifted into bits 4-7 of a 16-bit half is an IEEE
// half subnormal of value q*2^-20, a Q8 byte in bits 2-9 is q*2^-22: exact
// f16 operands (see the note at unpack() on why not bits 0-3). Activations
// are split x*2^-e = hi + lo into two f16 values (about 22 significant bits
// together, with a power-of-two scale 2^-e per RHS chosen from the block's
// max |x| so that neither part overflows or loses range); the matrix core multiplies
// exactly and accumulates in FP32. The scale factors 2^20 or 2^22 (code
// encoding) and 2^e (activation scale) are restored exactly in the FP32
// epilogue.
//
// Operands, code encoding and the tile product are in mfma_common.hpp.
//
// Work decomposition. A wave owns one 16-row tile and a contiguous range of
// K tiles; a workgroup holds RT waves (RT row tiles) over the same K range
// and stages that range of x once in LDS, already split into hi/lo f16 in
// MFMA operand order, with the per-group sums of x. A matrix is covered by
// nbands x ns workgroups (row bands x K splits). With ns > 1 each workgroup
// writes its partial sums to a workspace as 64-bit {value, epoch} slots; the
// last workgroup of a band to finish (an atomic counter elects it) takes the
// ns partials, each once its slot carries the launch's epoch, adds them in
// split order and writes y, so results do not depend on timing. Each lane keeps P entries of loads
// in flight in a register ring; the first P entries are requested before x is
// staged.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <mutex>
#include <type_traits>
#include <vector>

#include "kernels.hpp"
#include "mfma_common.hpp"

namespace qmr {
namespace {

using namespace mfma;

constexpr int kMaxRt = 8;
constexpr int kItems = 1;       // staged x slices per thread: tps * B * 16 <= kItems * 64 * rt
constexpr int kMetaUnits = 2;   // staged metadata loads per thread: ceil(tps*NGM/UE) <= 4 * kMetaUnits
constexpr uint32_t kMaxSplits = 32;  // K splits across workgroups

struct MfmaParams {
    const uint32_t *w;
    const void *s;
    const void *b;
    const float *x;
    float *y;
    unsigned long long *slots;  // [mat][ns][B][rows] {value, epoch} when ns > 1 or MLP
    uint32_t *counters;         // [nbands] when slots are used, zero between launches
    uint32_t rows, cols;
    uint32_t w_bytes, m_bytes;  // extents of the code and metadata views
    uint32_t nbands, ns, tiles, tps;
    const float *r;  // residual added to y in the final store (may alias y), or null
    // Fused MLP (w2 set): blocks nbands*ns.. take the up matrix (w2/s2/b2);
    // x is staged as x * norm; the last workgroup of a band adds both
    // matrices' partials and writes silu(gate/rms) * (up/rms).
    const uint32_t *w2;
    const void *s2;
    const void *b2;
    const float *norm;
    float eps;
    // Slot tags: partials are stored with `epoch`; the last arriver takes a
    // slot once it carries `wait_epoch` (the same, except under the testing
    // hook that forces a give-up), polling at most `spin_limit` times. A
    // slot still untagged then leaves NaN for its output and sets `status`
    // (0xC0000000 | band) for the host. With reset_slots the last arriver
    // stores zero into every slot it took, so a zeroed region stays zeroed.
    uint32_t epoch, wait_epoch, spin_limit;
    uint32_t *status;
    uint32_t reset_slots;
};

// FUSE 0: y = W x. FUSE 1: y = r + W x. FUSE 2: the fused MLP form. The
// fused forms are separate instances so that the plain product's code is
// untouched by them (runtime tests of their pointers cost the plain GEMV
// 0.6 us at the metric shape).
template <int BITS, int META, int GROUP, int B, int P, bool PAIRS, int FUSE>
__global__ __launch_bounds__(kMaxRt * 64) void affine_mfma_kernel(MfmaParams p) {
    constexpr int NGM = kTileK / GROUP;  // quant groups per tile
    constexpr int SLOTS = 16 / NGM;      // A rows per quant group
    constexpr int HALF = SLOTS / 2;      // RHS per quant group in D (>= B)
    constexpr int NLD = BITS / 4;        // 128-bit code loads per lane per tile
    constexpr int MB = META == 0 ? 4 : 2;
    constexpr int MW = META == 0 ? 2 : 1;  // LDS words per metadata entry
    constexpr int UE = PAIRS ? 2 : 1;      // entries per staged metadata load
    constexpr int LANE_BYTES = BITS * 4;   // code bytes of one K chunk (32 codes)
    constexpr int TPE = 8 / BITS;          // K tiles per 128-byte entry
    static_assert(2 * B <= SLOTS, "batch does not fit the slot layout");
    static_assert(!PAIRS || MB == 2, "paired metadata loads need 16-bit entries");

    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int r = lane & 15;
    const int lg = lane >> 4;
    const uint32_t RT = uint32_t(nthr) >> 6;
    constexpr bool mlp = FUSE == 2;
    const uint32_t nmat = mlp ? 2u : 1u;
    const uint32_t mat = mlp ? blockIdx.x / (p.nbands * p.ns) : 0u;
    const uint32_t bid = blockIdx.x - mat * p.nbands * p.ns;
    const uint32_t band = bid % p.nbands;
    const uint32_t split = bid / p.nbands;
    const uint32_t T0 = split * p.tps;
    const uint32_t T1 = min(T0 + p.tps, p.tiles);
    const uint32_t nT = T1 - T0;
    const uint32_t G = nT * NGM;                    // metadata entries per row in this split
    const uint32_t Gp = (p.tps * NGM + 1) | 1;      // their LDS pitch (odd: spreads banks)
    const uint32_t band_row0 = band * RT * 16;

    u4 *ldsA = reinterpret_cast<u4 *>(lds);  // [tps][4 m][4 g][2B] operand blocks
    float4 *ldsSx = reinterpret_cast<float4 *>(lds + size_t(p.tps) * 4 * 4 * 2 * B * 16);
    // ldsSx [tps][NGM][HALF/2]: (sum x_t, sum x_t+1, 2^(c+e_t), 2^(c+e_t+1)) per RHS pair
    uint32_t *ldsM = reinterpret_cast<uint32_t *>(ldsSx + size_t(p.tps) * NGM * (HALF / 2));
    // ldsM [RT*16 rows][Gp] entries: s | b << 16 (16-bit) or (s, b) as two words
    int *ldsLast = reinterpret_cast<int *>(ldsM + size_t(RT) * 16 * Gp * MW);

    const uint32_t tile0 = band_row0 + wave * 16;

    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t *>(mat ? p.w2 : p.w), 0, int(p.w_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(mat ? p.s2 : p.s), 0, int(p.m_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t br =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(mat ? p.b2 : p.b), 0, int(p.m_bytes), kRsrcWord3);

    // ---- 1. Metadata of the band's rows over this K range (to LDS below). ----
    // Rows past the matrix read zeros through the buffer range check.
    const uint32_t m_pitch = p.cols / GROUP;
    const uint32_t units_per_row = (G + UE - 1) / UE;
    const uint32_t units = RT * 16 * units_per_row;
    // Loads are issued only by waves that have work (a wave-uniform test), so
    // idle lanes do not queue memory instructions ahead of the weight ring.
    const uint32_t wave_base = __builtin_amdgcn_readfirstlane(uint32_t(tid) & ~63u);
    uint32_t mv_s[kMetaUnits], mv_b[kMetaUnits];
#pragma unroll
    for (int u = 0; u < kMetaUnits; ++u) {
        mv_s[u] = mv_b[u] = 0u;
        if (wave_base + u * nthr >= units) continue;
        const uint32_t f = tid + u * nthr;
        const uint32_t rl = f / units_per_row;
        const uint32_t gu = f - rl * units_per_row;
        const uint32_t off = f < units ? ((band_row0 + rl) * m_pitch + T0 * NGM + gu * UE) * MB : kOut;
        if constexpr (MB == 4 || PAIRS) {
            mv_s[u] = __builtin_amdgcn_raw_buffer_load_b32(sr, int(off), 0, 0);
            mv_b[u] = __builtin_amdgcn_raw_buffer_load_b32(br, int(off), 0, 0);
        } else {
            mv_s[u] = __builtin_amdgcn_raw_buffer_load_b16(sr, int(off), 0, 0);
            mv_b[u] = __builtin_amdgcn_raw_buffer_load_b16(br, int(off), 0, 0);
        }
    }

    // ---- 2. This thread's slices of x. Item = (tile Tl, RHS t, K chunk g,
    // MFMA m): 8 consecutive columns; the GROUP/8 items of one quant group sit
    // in consecutive lanes. ----
    const uint32_t items = nT * B * 16;
    // x is read through a buffer view; slices past cols (a K tail) or past
    // the item count are sent to kOut and read as zeros.
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(p.x), 0, int(uint32_t(B) * p.cols * 4u), kRsrcWord3);
    float xv[kItems][8];
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[i][j] = 0.f;
        if (wave_base + i * nthr >= items) continue;
        const uint32_t it = tid + i * nthr;
        load_x8(xv[i], xr, uint32_t(item_pos<B>(it).t), T0 * kTileK + item_col<B>(it), p.cols, it < items);
        if constexpr (mlp) {
            const __amdgpu_buffer_rsrc_t nr = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(p.norm), 0, int(p.cols * 4u), kRsrcWord3);
            float nv[8];
            load_x8(nv, nr, 0u, T0 * kTileK + item_col<B>(it), p.cols, it < items);
#pragma unroll
            for (int j = 0; j < 8; ++j) xv[i][j] *= nv[j];
        }
    }

    // ---- 3. The first P entries of codes, requested in ring order. ----
    // An entry is 128 contiguous bytes of each of the wave's 16 rows (TPE
    // K tiles), read with two 128-bit loads per lane: the first covers rows
    // 0-7 and the second rows 8-15, eight lanes per row. A lane (r, g) keeps
    // the piece of its own row that the MFMA layout gives it (kp) and fetches
    // for lane r^8 the piece that lane needs from the other half (sp); the
    // two swap through DPP after the loads land.
    const uint32_t row = band_row0 + wave * 16 + r;
    const bool row_ok = row < p.rows;
    const bool lo_half = r < 8;
    const uint32_t kp = BITS == 4 ? uint32_t(lg) : 2u * lg;       // 16-byte piece kept
    const uint32_t sp = BITS == 4 ? uint32_t(lg) + 4 : 2u * lg + 1;  // piece sent to lane r^8
    const uint32_t piece1 = lo_half ? kp : sp;  // load 1 (rows 0-7)
    const uint32_t piece2 = lo_half ? sp : kp;  // load 2 (rows 8-15)
    const uint32_t row_bytes = p.cols / 32 * LANE_BYTES;
    const uint32_t base1 = (tile0 + (r & 7)) * row_bytes + 16 * piece1;
    const uint32_t base2 = (tile0 + 8 + (r & 7)) * row_bytes + 16 * piece2;
    // Bytes of each row this split may read: min(row end, split end).
    const uint32_t end_b = min(row_bytes, T1 * (4 * LANE_BYTES));
    const uint32_t E0 = T0 / TPE;  // first entry (tps is a multiple of TPE)
    auto issue = [&](u4 (&c)[2], uint32_t E) {
        const uint32_t eb = E * 128;
        const uint32_t o1 = eb + 16 * piece1 < end_b ? base1 + eb : kOut;
        const uint32_t o2 = eb + 16 * piece2 < end_b ? base2 + eb : kOut;
        c[0] = __builtin_amdgcn_raw_buffer_load_b128(wr, int(o1), 0, kAuxStream);
        c[1] = __builtin_amdgcn_raw_buffer_load_b128(wr, int(o2), 0, kAuxStream);
    };
    u4 ring[P][2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < P; ++j) {
        issue(ring[j], E0 + j);
        __builtin_amdgcn_sched_barrier(0);
    }


    // ---- 4. Metadata to LDS (waits only for the metadata loads). ----
#pragma unroll
    for (int u = 0; u < kMetaUnits; ++u) {
        const uint32_t f = tid + u * nthr;
        if (f < units) {
            const uint32_t rl = f / units_per_row;
            const uint32_t gu = f - rl * units_per_row;
            uint32_t *dst = ldsM + (rl * Gp + gu * UE) * MW;
            if constexpr (MB == 4) {
                dst[0] = mv_s[u];
                dst[1] = mv_b[u];
            } else if constexpr (PAIRS) {
                dst[0] = __builtin_amdgcn_perm(mv_b[u], mv_s[u], 0x05040100u);
                dst[1] = __builtin_amdgcn_perm(mv_b[u], mv_s[u], 0x07060302u);
            } else {
                dst[0] = (mv_s[u] & 0xFFFFu) | (mv_b[u] << 16);
            }
        }
    }

    // ---- 5. x as MFMA A operands (hi/lo f16, group sums, epilogue factors). ----
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const uint32_t it = tid + i * nthr;
        if (i > 0 && it >= items) break;  // whole 16-lane blocks are in or out
        stage_x_item<BITS, GROUP, B>(xv[i], it, it < items, lane, ldsA, ldsSx);
    }
    stage_x_pads<GROUP, B>(nT, tid, nthr, ldsSx);
    lds_barrier();

    // ---- 6. Per-lane constants of the A operand and the D epilogue. ----
    const LaneMap<GROUP, B> L(lane);
    const int t0 = L.t0;
    const uint32_t m_idx = (uint32_t(wave) * 16 + r) * Gp + uint32_t(L.gD);

    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    h8 a[4] = {h8{}, h8{}, h8{}, h8{}};
    auto compute = [&](const u4 (&c)[NLD], uint32_t Tl) {
        float sv, bv;
        meta_entry<META>(ldsM + (m_idx + Tl * NGM) * MW, sv, bv);
        const float4 sx = ldsSx[(Tl * NGM + L.gD) * (HALF / 2) + t0 / 2];
        tile_product<BITS, META, GROUP, B>(c, L, ldsA + Tl * 4 * (8 * B), sv, bv, sx, a, acc);
    };

    // Swap the pieces of lanes r and r^8 (DPP row rotate by 8 inside each
    // 16-lane row): afterwards kept = piece kp and got = piece sp of row r.
    auto exchange = [&](const u4 (&c)[2], u4 &kept, u4 &got) {
        u4 send;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            kept[d] = lo_half ? c[0][d] : c[1][d];
            send[d] = lo_half ? c[1][d] : c[0][d];
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) got[d] = uint32_t(__builtin_amdgcn_mov_dpp(int(send[d]), 0x128, 0xF, 0xF, false));
    };

    // ---- 7. Stream the K range. Loads are issued unconditionally (past the
    // range they read zeros and move no data), so the ring registers never
    // merge across branches and each entry waits only for its own loads. ----
    const uint32_t nE = (nT + TPE - 1) / TPE;
    for (uint32_t base = 0; base < nE; base += P) {
#pragma unroll
        for (int j = 0; j < P; ++j) {
            const uint32_t E = base + j;
            if (E < nE) {
                u4 kept, got;
                exchange(ring[j], kept, got);
                if constexpr (BITS == 4) {
                    const u4 c0[1] = {kept};
                    compute(c0, E * 2);
                    if (E * 2 + 1 < nT) {
                        const u4 c1[1] = {got};
                        compute(c1, E * 2 + 1);
                    }
                } else {
                    const u4 c[2] = {kept, got};
                    compute(c, E);
                }
            }
            issue(ring[j], E0 + E + P);
        }
    }

    // ---- 8. Combine hi/lo slots and quant groups; write y or a partial. ----
    float v0, v1;
    combine_slots<GROUP>(acc, v0, v1);
    constexpr int WRITERS = 4 / NGM;  // lane groups holding distinct RHS pairs
    const bool writer = lg < WRITERS && row_ok;
    if (p.ns == 1 && !mlp) {
        if (writer) {
            const size_t o0 = size_t(t0) * p.rows + row, o1 = o0 + p.rows;
            if (t0 < B) p.y[o0] = FUSE == 1 ? p.r[o0] + v0 : v0;
            if (t0 + 1 < B) p.y[o1] = FUSE == 1 ? p.r[o1] + v1 : v1;
        }
        return;
    }
    // Split K: publish this split's partial sums as {value, epoch} slots;
    // the last workgroup of the band to arrive adds the ns partials in split
    // order. The arrival counter only elects that workgroup: a partial counts
    // once its slot's 64-bit word (one single-copy-atomic store) carries the
    // launch's epoch, so the sum does not depend on when the other splits'
    // stores become visible relative to their counter increments. Every
    // other split incremented the counter after issuing its stores, so the
    // last arriver's wait ends as soon as they land.
    unsigned long long *part = p.slots + size_t(mat * p.ns + split) * B * p.rows;
    const unsigned long long tag = (unsigned long long)p.epoch << 32;
    if (writer) {
        if (t0 < B)
            __hip_atomic_store(part + size_t(t0) * p.rows + row, tag | __float_as_uint(v0), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if (t0 + 1 < B)
            __hip_atomic_store(part + size_t(t0 + 1) * p.rows + row, tag | __float_as_uint(v1), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&p.counters[band], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *ldsLast = prev == nmat * p.ns - 1 ? 1 : 0;
    }
    __syncthreads();
    if (*ldsLast == 0) return;
    const uint32_t band_rows = RT * 16;
    // MLP: 1/rms of each x[t] (the staged x carried the norm weights only),
    // from sum(x^2) over all columns, reduced through LDS (the operand area
    // is free once every wave has left the main loop).
    float inv[B];
#pragma unroll
    for (int t = 0; t < B; ++t) inv[t] = 1.f;
    if constexpr (mlp) {
        float *sq = reinterpret_cast<float *>(lds);
#pragma unroll
        for (int t = 0; t < B; ++t) {
            float v = 0.f;
            for (uint32_t k = uint32_t(tid) * 4u; k < p.cols; k += uint32_t(nthr) * 4u) {
                const u4 q = __builtin_amdgcn_raw_buffer_load_b128(xr, int((uint32_t(t) * p.cols + k) * 4u), 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e) v += __uint_as_float(q[e]) * __uint_as_float(q[e]);
            }
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
            if (lane == 0) sq[wave * B + t] = v;
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < B; ++t) {
            float ss = 0.f;
            for (uint32_t wv = 0; wv < RT; ++wv) ss += sq[wv * B + t];
            inv[t] = 1.0f / sqrtf(ss / float(p.cols) + p.eps);
        }
    }
    bool ok = true;
    // The sum of one matrix's ns partials at slot `first` (stride apart), in
    // split order: chunks of eight loads in flight, each slot polled until it
    // carries the launch's epoch.
    auto take = [&](unsigned long long *first, size_t stride) {
        constexpr uint32_t kChunk = 8;
        float v = 0.f;
        for (uint32_t k0 = 0; k0 < p.ns; k0 += kChunk) {
            unsigned long long w[kChunk];
#pragma unroll
            for (uint32_t k = 0; k < kChunk; ++k)
                w[k] = k0 + k < p.ns ? __hip_atomic_load(first + (k0 + k) * stride, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT)
                                     : 0ull;
#pragma unroll
            for (uint32_t k = 0; k < kChunk; ++k) {
                if (k0 + k >= p.ns) break;
                unsigned long long *slot = first + (k0 + k) * stride;
                for (uint32_t spins = 0; uint32_t(w[k] >> 32) != p.wait_epoch;) {
                    if (++spins > p.spin_limit) {
                        ok = false;
                        w[k] = 0x7FC00000ull;  // NaN
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                    w[k] = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                v += __uint_as_float(uint32_t(w[k]));
                if (p.reset_slots) __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        return v;
    };
    const size_t stride = size_t(B) * p.rows;
    for (uint32_t i = tid; i < band_rows * B; i += nthr) {
        const uint32_t t = i / band_rows;
        const uint32_t rr = band_row0 + i % band_rows;
        if (rr >= p.rows) continue;
        const size_t o = size_t(t) * p.rows + rr;
        const float v = take(p.slots + o, stride);
        if constexpr (mlp) {
            // The up matrix's partials follow the gate's ns blocks.
            const float u = take(p.slots + size_t(p.ns) * stride + o, stride);
            float it = inv[0];
#pragma unroll
            for (int tt = 1; tt < B; ++tt) it = uint32_t(tt) == t ? inv[tt] : it;
            const float g = v * it;
            p.y[o] = g * (1.0f / (1.0f + expf(-g))) * (u * it);
        } else {
            p.y[o] = FUSE == 1 ? p.r[o] + v : v;
        }
    }
    if (!ok && p.status)
        __hip_atomic_store(p.status, 0xC0000000u | band, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (tid == 0) __hip_atomic_store(&p.counters[band], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kRing = 2;  // entries in flight per wave

template <int BITS, int META, int GROUP, int B, bool PAIRS>
hipError_t launch_b(const MfmaParams &p, uint32_t rt, size_t lds, hipStream_t stream) {
    const int fuse = p.w2 ? 2 : p.r ? 1 : 0;
    auto kernel = fuse == 2   ? affine_mfma_kernel<BITS, META, GROUP, B, kRing, PAIRS, 2>
                  : fuse == 1 ? affine_mfma_kernel<BITS, META, GROUP, B, kRing, PAIRS, 1>
                              : affine_mfma_kernel<BITS, META, GROUP, B, kRing, PAIRS, 0>;
    if (lds > 65536) {
        const hipError_t e = raise_lds_limit(reinterpret_cast<const void *>(kernel), lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, dim3(p.nbands * p.ns * (p.w2 ? 2u : 1u)), dim3(rt * 64), lds, stream, p);
    return hipGetLastError();
}

template <int BITS, int META, int GROUP, int B>
hipError_t launch_pairs(const MfmaParams &p, bool pairs, uint32_t rt, size_t lds, hipStream_t stream) {
    if constexpr (META != 0) {
        if (pairs) return launch_b<BITS, META, GROUP, B, true>(p, rt, lds, stream);
    }
    return launch_b<BITS, META, GROUP, B, false>(p, rt, lds, stream);
}

template <int BITS, int META, int GROUP>
hipError_t launch_group(const MfmaParams &p, uint32_t batch, bool pairs, uint32_t rt, size_t lds,
                        hipStream_t stream) {
    constexpr int MAXB = (16 / (kTileK / GROUP)) / 2;
    switch (batch) {
        case 1: return launch_pairs<BITS, META, GROUP, 1>(p, pairs, rt, lds, stream);
        case 2: return launch_pairs<BITS, META, GROUP, 2>(p, pairs, rt, lds, stream);
        case 3:
            if constexpr (MAXB >= 3) return launch_pairs<BITS, META, GROUP, 3>(p, pairs, rt, lds, stream);
            break;
        case 4:
            if constexpr (MAXB >= 4) return launch_pairs<BITS, META, GROUP, 4>(p, pairs, rt, lds, stream);
            break;
        default: break;
    }
    return hipErrorInvalidValue;
}

template <int BITS, int META>
hipError_t launch_meta(const MfmaParams &p, uint32_t group, uint32_t batch, bool pairs, uint32_t rt,
                       size_t lds, hipStream_t stream) {
    switch (group) {
        case 32: return launch_group<BITS, META, 32>(p, batch, pairs, rt, lds, stream);
        case 64: return launch_group<BITS, META, 64>(p, batch, pairs, rt, lds, stream);
        case 128: return launch_group<BITS, META, 128>(p, batch, pairs, rt, lds, stream);
        default: return hipErrorInvalidValue;
    }
}

// The kernel instance for a format, for occupancy queries (the plain form's;
// the fused forms plan with its occupancy).
template <int BITS, int META, int GROUP>
const void *instance_group(uint32_t batch, bool pairs) {
    constexpr int MAXB = (16 / (kTileK / GROUP)) / 2;
    auto pick = [&](auto bconst) -> const void * {
        constexpr int B = decltype(bconst)::value;
        if constexpr (META != 0) {
            if (pairs) return reinterpret_cast<const void *>(affine_mfma_kernel<BITS, META, GROUP, B, kRing, true, 0>);
        }
        return reinterpret_cast<const void *>(affine_mfma_kernel<BITS, META, GROUP, B, kRing, false, 0>);
    };
    switch (batch) {
        case 1: return pick(std::integral_constant<int, 1>{});
        case 2: return pick(std::integral_constant<int, 2>{});
        case 3:
            if constexpr (MAXB >= 3) return pick(std::integral_constant<int, 3>{});
            break;
        case 4:
            if constexpr (MAXB >= 4) return pick(std::integral_constant<int, 4>{});
            break;
        default: break;
    }
    return nullptr;
}

template <int BITS, int META>
const void *instance_meta(uint32_t group, uint32_t batch, bool pairs) {
    switch (group) {
        case 32: return instance_group<BITS, META, 32>(batch, pairs);
        case 64: return instance_group<BITS, META, 64>(batch, pairs);
        case 128: return instance_group<BITS, META, 128>(batch, pairs);
        default: return nullptr;
    }
}

const void *instance(const AffineArgs &a, bool pairs) {
    const int meta = static_cast<int>(a.meta);
    if (a.bits == 4) {
        if (meta == 0) return instance_meta<4, 0>(a.group, a.batch, false);
        if (meta == 1) return instance_meta<4, 1>(a.group, a.batch, pairs);
        return instance_meta<4, 2>(a.group, a.batch, pairs);
    }
    if (meta == 0) return instance_meta<8, 0>(a.group, a.batch, false);
    if (meta == 1) return instance_meta<8, 1>(a.group, a.batch, pairs);
    return instance_meta<8, 2>(a.group, a.batch, pairs);
}

// Resident workgroups per CU for a kernel instance, block size and dynamic
// LDS (as the runtime computes it from registers and LDS); cached.
uint32_t resident_per_cu(const void *kernel, uint32_t threads, size_t lds) {
    struct Entry {
        const void *k;
        uint32_t threads;
        size_t lds;
        uint32_t n;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry &e : cache)
        if (e.k == kernel && e.threads == threads && e.lds == lds) return e.n;
    int n = 0;
    if (kernel == nullptr ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, int(threads), lds) != hipSuccess || n < 1)
        n = 1;
    cache.push_back(Entry{kernel, threads, lds, uint32_t(n)});
    return uint32_t(n);
}

}  // namespace

size_t mfma_lds_bytes(uint32_t tps, uint32_t ngm, uint32_t batch, uint32_t rt, bool f32_meta) {
    const size_t gp = ((size_t(tps) * ngm + 1) | 1);
    return size_t(tps) * (4 * 4 * 2 * batch * 16 + 64) + size_t(rt) * 16 * gp * 4 * (f32_meta ? 2 : 1) + 16;
}

MfmaPlan plan_affine_mfma(const AffineArgs &a, const DeviceLimits &lim, uint32_t force_ns) {
    MfmaPlan pl;
    if (!affine_mfma_supported(a)) return pl;
    const uint32_t ngm = kTileK / a.group;
    const uint32_t row_tiles = (a.rows + 15) / 16;
    const uint32_t tiles = (a.cols + kTileK - 1) / kTileK;
    const bool f32_meta = a.meta == Meta::F32;
    pl.rt = row_tiles < uint32_t(kMaxRt) ? row_tiles : uint32_t(kMaxRt);
    pl.nbands = (row_tiles + pl.rt - 1) / pl.rt;
    // Paired (32-bit) metadata loads need every row's run to start on an even
    // entry: even groups per row and an even number of groups per split.
    const bool pairs_ok = !f32_meta && (a.cols / a.group) % 2 == 0;
    // Per-thread staging bounds: x slices (tps * B <= 4 * kItems * rt) and
    // metadata loads (tps * NGM <= 4 * kMetaUnits * entries per load).
    const uint32_t cap_x = 4u * kItems * pl.rt / a.batch;
    // K splits: aim for about twenty waves per CU (short K ranges stream
    // best here: every wave's whole range is requested within two ring
    // refills) with equal K ranges, and never more workgroups than stay
    // resident at once (a second round would add a whole wave of latency).
    // Score = |log(waves/target)| plus twice the log of the split imbalance.
    const uint32_t cus = lim.num_cus > 0 ? uint32_t(lim.num_cus) : 256u;
    double best = 1e30;
    uint32_t best_resident = 1;
    const uint32_t tpe = 8 / a.bits;  // K tiles per 128-byte load entry
    for (uint32_t ns = 1; ns <= tiles && ns <= kMaxSplits; ++ns) {
        if (force_ns && ns != force_ns) continue;
        uint32_t tps = (tiles + ns - 1) / ns;
        tps = (tps + tpe - 1) / tpe * tpe;  // splits start on an entry
        const uint32_t eff = (tiles + tps - 1) / tps;
        const bool pairs = pairs_ok && (tps * ngm) % 2 == 0;
        const uint32_t cap_m = 4u * kMetaUnits * (pairs ? 2u : 1u) / ngm;
        if (tps > cap_x || tps > cap_m || eff != ns) continue;
        const size_t lds = mfma_lds_bytes(tps, ngm, a.batch, pl.rt, f32_meta);
        if (lds > lim.max_lds_per_block) continue;
        const uint32_t resident = resident_per_cu(instance(a, pairs), pl.rt * 64, lds) * cus;
        const double target = std::min(20.0, double(resident / cus) * pl.rt) * cus;
        // The fused MLP form runs the gate and up matrices in one grid.
        const uint32_t nmat = a.up_w ? 2u : 1u;
        const double waves = double(pl.nbands) * pl.rt * eff * nmat;
        double score = std::fabs(std::log(waves / target)) + 2.0 * std::log(double(tps) * eff / double(tiles));
        if (pl.nbands * eff * nmat > resident)
            score += 10.0 * std::ceil(double(pl.nbands * eff * nmat) / resident);
        if (score < best - 1e-9) {
            best = score;
            pl.tps = tps;
            pl.ns = eff;
            pl.pairs = pairs;
            best_resident = resident > 0 ? resident : 1;
        }
    }
    if (pl.ns == 0) {
        if (force_ns) return plan_affine_mfma(a, lim, 0);  // infeasible forced count: the planner's
        pl.rt = 0;
        return pl;
    }
    pl.tiles = tiles;
    pl.lds = mfma_lds_bytes(pl.tps, ngm, a.batch, pl.rt, f32_meta);
    pl.rounds = (pl.nbands * pl.ns * (a.up_w ? 2u : 1u) + best_resident - 1) / best_resident;
    return pl;
}

bool affine_mfma_supported(const AffineArgs &a) {
    if (a.bits != 4 && a.bits != 8) return false;
    if (a.group != 32 && a.group != 64 && a.group != 128) return false;
    const uint32_t maxb = (16 / (kTileK / a.group)) / 2;
    if (a.batch < 1 || a.batch > maxb) return false;
    if (a.cols % 32 != 0 || a.cols % a.group != 0) return false;
    if ((reinterpret_cast<uintptr_t>(a.w) & 15) != 0) return false;
    const uint64_t w_bytes = uint64_t(a.rows) * a.cols * a.bits / 8;
    const uint64_t m_bytes = uint64_t(a.rows) * (a.cols / a.group) * (a.meta == Meta::F32 ? 4 : 2);
    return w_bytes < (1ull << 31) && m_bytes < (1ull << 31);
}

size_t affine_mfma_workspace(const MfmaPlan &pl, const AffineArgs &a) {
    // The fused MLP form always publishes partials (gate and up meet in the
    // band's last workgroup), one set per matrix, as 64-bit slots.
    if (pl.ns <= 1 && !a.up_w) return 0;
    return size_t(a.up_w ? 2 : 1) * pl.ns * a.batch * a.rows * sizeof(unsigned long long);
}

hipError_t launch_affine_mfma(const AffineArgs &a, const MfmaPlan &pl, unsigned long long *slots,
                              uint32_t *counters, uint32_t epoch, const TileWait &wait, hipStream_t stream) {
    MfmaParams p;
    p.w = a.w;
    p.s = a.s;
    p.b = a.b;
    p.x = a.x;
    p.y = a.y;
    p.r = a.residual;
    p.w2 = a.up_w;
    p.s2 = a.up_s;
    p.b2 = a.up_b;
    p.norm = a.norm;
    p.eps = a.eps;
    p.slots = slots;
    p.counters = counters;
    p.epoch = epoch;
    p.wait_epoch = wait.force_give_up ? epoch + 0x40000000u : epoch;
    p.spin_limit = wait.force_give_up ? 64u : 1u << 22;
    p.status = wait.status;
    p.reset_slots = wait.reset_slots ? 1u : 0u;
    p.rows = a.rows;
    p.cols = a.cols;
    p.w_bytes = uint32_t(uint64_t(a.rows) * a.cols * a.bits / 8);
    p.m_bytes = uint32_t(uint64_t(a.rows) * (a.cols / a.group) * (a.meta == Meta::F32 ? 4 : 2));
    p.nbands = pl.nbands;
    p.ns = pl.ns;
    p.tiles = pl.tiles;
    p.tps = pl.tps;
    const int meta = static_cast<int>(a.meta);
    if (a.bits == 4) {
        if (meta == 0) return launch_meta<4, 0>(p, a.group, a.batch, false, pl.rt, pl.lds, stream);
        if (meta == 1) return launch_meta<4, 1>(p, a.group, a.batch, pl.pairs, pl.rt, pl.lds, stream);
        return launch_meta<4, 2>(p, a.group, a.batch, pl.pairs, pl.rt, pl.lds, stream);
    }
    if (meta == 0) return launch_meta<8, 0>(p, a.group, a.batch, false, pl.rt, pl.lds, stream);
    if (meta == 1) return launch_meta<8, 1>(p, a.group, a.batch, pl.pairs, pl.rt, pl.lds, stream);
    return launch_meta<8, 2>(p, a.group, a.batch, pl.pairs, pl.rt, pl.lds, stream);
}

}  // namespace qmr

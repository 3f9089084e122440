// Dense F16 products on the matrix cores (matvec_f16 / matmul_f16, batch 1..4):
//     y[t*rows + r] = sum_c w[r,c] * x[t,c]
// the reference's dense kernels (kernels/qwen.metal:48-57,
// kernels/matmul_block.metal:213-248), F16 weights times FP32 x.
//
// Exactness. F16 weights are MFMA operands as stored. x is split into hi/lo
// f16 parts with a power-of-two scale per (128-column tile, RHS), as in the
// quantized kernels (mfma_common.hpp: about 22 significant bits together);
// the matrix core multiplies exactly and accumulates in FP32, and the FP32
// epilogue restores the scale.
//
// Work decomposition. Grid = row bands x K splits, blockIdx = band +
// nbands * split. A workgroup holds RT x KW waves: RT 16-row tiles, each
// split again into KW contiguous runs of the split's 128-column tiles, one
// wave per run. It stages the split's x once in LDS as MFMA A operand
// images, shared by all its waves, and each wave streams its run's 128-byte
// entries (two per 128-column tile) through a register ring of P entries:
// the first 16-byte load of a lane covers rows 0-7 and the second rows 8-15,
// eight lanes per 128-byte row segment, and lanes r and r^8 swap one piece
// through DPP. After the swap lane (r, g) holds pieces g and g+4 of each
// entry of row r, so MFMA m of a tile takes the tile's piece 4m + g: x item
// (tile, RHS, g, m) is staged from columns 32m + 8g .. +8 of the tile. The
// KW runs of a tile are added in run order through LDS.
//
// With ns > 1 every workgroup publishes its sums as 64-bit {value, epoch}
// slots and the band's last workgroup to arrive (an arrival counter elects
// it) takes each slot once it carries the launch's epoch and adds them in
// split order, so results do not depend on timing and no workgroup waits for
// one that is not resident (plans may span several rounds).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <mutex>
#include <vector>

#include "kernels.hpp"
#include "mfma_common.hpp"

namespace qmr {
namespace {

using namespace mfma;

constexpr int kMaxWaves = 8;
constexpr uint32_t kMaxDenseSplits = 32;
constexpr int kGroup = 128;      // one x scale per 128-column tile and RHS
constexpr int kDppRor8 = 0x128;  // row_ror:8: lane i <- lane i ^ 8 within 16 lanes
// Planner cost model (microseconds; see dense_cost), fitted on MI355X to
// 2535 timed plans over four shapes (2048..17408 rows, 5120..17408 columns)
// and 1..4 RHS: rms error 8% (log scale), and the plan it picks is on
// average within 5% of the fastest plan timed.
constexpr double kDenseStartUs = 2.16;     // launch, first loads, x staging
constexpr double kDenseLatencyUs = 0.86;   // one ring refill of a wave
constexpr double kDenseBytesPerUs = 8.1e6; // streaming rate of evenly loaded CUs
constexpr double kDenseXCost = 1.05;       // staged x bytes, relative to weight bytes
constexpr double kDenseRoundUs = 3.0;      // each further round of resident workgroups
constexpr double kDenseElectUs = 1.29;     // split plans: arrival election
constexpr double kDenseSlotUs = 1.67;      // and each eight slots per output

struct DenseParams {
    const uint16_t *w;
    const float *x;
    float *y;
    unsigned long long *slots;  // [ns][B][rows] {value, epoch} when ns > 1
    uint32_t *counters;         // [nbands] when ns > 1, zero between launches
    uint32_t rows, cols, w_bytes;
    uint32_t nbands, ns, tiles, tps, kw;
    // Slot tags and the finisher's bounded wait (as in the split-K kernel):
    // a slot counts once it carries wait_epoch; past spin_limit polls the
    // output is NaN and status gets 0xA0000000 | band.
    uint32_t epoch, wait_epoch, spin_limit;
    uint32_t *status;
    uint32_t reset_slots;
};

// First column of x item it (tile Tl, RHS t, lane group g, MFMA m) relative
// to the split's first column: the piece that lane group g of MFMA m holds.
template <int B>
__device__ __forceinline__ uint32_t dense_item_col(uint32_t it) {
    const ItemPos q = item_pos<B>(it);
    return q.Tl * kTileK + 32u * q.m + 8u * q.g;
}

template <int B, int XI, int P>
__global__ __launch_bounds__(kMaxWaves * 64) void dense_mfma_kernel(DenseParams p) {
    constexpr int HALF = 16 / 2;  // RHS per slot group of D (one x scale group per tile)
    static_assert(2 * B <= 16, "batch does not fit the slot layout");
    static_assert(P % 2 == 0, "the ring holds whole tiles");

    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const uint32_t wave = uint32_t(__builtin_amdgcn_readfirstlane(tid >> 6));
    const int lane = tid & 63;
    const int r = lane & 15;
    const int lg = lane >> 4;
    const uint32_t KW = p.kw;
    const uint32_t RT = (uint32_t(nthr) >> 6) / KW;
    const uint32_t wtile = wave / KW, kq = wave % KW;
    const uint32_t band = blockIdx.x % p.nbands;
    const uint32_t split = blockIdx.x / p.nbands;
    const uint32_t T0 = split * p.tps;
    const uint32_t T1 = min(T0 + p.tps, p.tiles);
    const uint32_t nT = T1 - T0;
    const uint32_t band_row0 = band * RT * 16u;
    const uint32_t tile0 = band_row0 + wtile * 16u;
    // This wave's run of the split's tiles: [Ta, Tb).
    const uint32_t tpw = (nT + KW - 1) / KW;
    const uint32_t Ta = min(kq * tpw, nT), Tb = min(Ta + tpw, nT);

    u4 *ldsA = reinterpret_cast<u4 *>(lds);  // [tps][4 m][4 g][2B] operand blocks
    float4 *ldsSx = reinterpret_cast<float4 *>(lds + size_t(p.tps) * 4 * 4 * 2 * B * 16);  // [tps][HALF/2]
    float2 *ldsRed = reinterpret_cast<float2 *>(ldsSx + size_t(p.tps) * (HALF / 2));      // [waves][64]
    int *ldsLast = reinterpret_cast<int *>(ldsRed + nthr);

    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(p.w), 0, int(p.w_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(p.x), 0, int(uint32_t(B) * p.cols * 4u), kRsrcWord3);

    // ---- 1. The split's x, requested first. ----
    const uint32_t items = nT * B * 16u;
    const uint32_t wave_base = wave * 64u;
    float xv[XI][8];
#pragma unroll
    for (int i = 0; i < XI; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[i][j] = 0.f;
        if (wave_base + uint32_t(i * nthr) >= items) continue;
        const uint32_t it = uint32_t(tid) + uint32_t(i * nthr);
        load_x8(xv[i], xr, uint32_t(item_pos<B>(it).t), T0 * kTileK + dense_item_col<B>(it), p.cols, it < items);
    }

    // ---- 2. The first P entries of the run's rows. ----
    const uint32_t row_bytes = p.cols * 2u;
    const bool lo_half = r < 8;
    const uint32_t kp = uint32_t(lg);      // 16-byte piece kept
    const uint32_t sp = uint32_t(lg) + 4;  // piece sent to lane r^8
    const uint32_t piece1 = lo_half ? kp : sp;
    const uint32_t piece2 = lo_half ? sp : kp;
    const uint32_t rowA = tile0 + uint32_t(r & 7), rowB = tile0 + 8u + uint32_t(r & 7);
    const uint32_t eb0 = (T0 + Ta) * 256u;  // the run's first byte within a row
    const uint32_t nE = (Tb - Ta) * 2u;     // entries of the run
    // Entry E of the run; past the run or a row's end the pieces read zeros
    // through the out-of-range offset.
    const uint32_t vA = rowA < p.rows ? rowA * row_bytes + eb0 + 16u * piece1 : kOut;
    const uint32_t vB = rowB < p.rows ? rowB * row_bytes + eb0 + 16u * piece2 : kOut;
    // Bytes of the row from the run's first piece of each load on (0 when
    // the row ends before it).
    const uint32_t endA = eb0 + 16u * piece1 < row_bytes ? row_bytes - eb0 - 16u * piece1 : 0u;
    const uint32_t endB = eb0 + 16u * piece2 < row_bytes ? row_bytes - eb0 - 16u * piece2 : 0u;
    auto issue = [&](u4 (&c)[2], uint32_t E) {
        const uint32_t eo = E * 128u;
        const bool live = E < nE;
        const uint32_t o1 = live && vA != kOut && eo < endA ? vA + eo : kOut;
        const uint32_t o2 = live && vB != kOut && eo < endB ? vB + eo : kOut;
        c[0] = __builtin_amdgcn_raw_buffer_load_b128(wr, int(o1), 0, kAuxStream);
        c[1] = __builtin_amdgcn_raw_buffer_load_b128(wr, int(o2), 0, kAuxStream);
    };
    u4 ring[P][2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < P; ++j) {
        issue(ring[j], uint32_t(j));
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- 3. x as MFMA A operands (hi/lo f16, epilogue factors). ----
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const uint32_t it = uint32_t(tid) + uint32_t(i * nthr);
        if (i > 0 && it >= items) break;  // whole 16-lane blocks are in or out
        stage_x_item<16, kGroup, B>(xv[i], it, it < items, lane, ldsA, ldsSx);
    }
    stage_x_pads<kGroup, B>(nT, tid, nthr, ldsSx);
    lds_barrier();

    // ---- 4. Stream the run. ----
    const LaneMap<kGroup, B> L(lane);
    const int t0 = L.t0;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    h8 a[4] = {h8{}, h8{}, h8{}, h8{}};
    auto exchange = [&](const u4 (&c)[2], u4 &kept, u4 &got) {
        u4 send;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            kept[d] = lo_half ? c[0][d] : c[1][d];
            send[d] = lo_half ? c[1][d] : c[0][d];
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) got[d] = dpp_u32<kDppRor8>(send[d]);
    };
    auto tile = [&](const u4 (&b)[4], uint32_t Tl) {
        const u4 *img = ldsA + Tl * 4u * (8u * B);
        if (L.a_ok) {
#pragma unroll
            for (int m = 0; m < 4; ++m) a[m] = __builtin_bit_cast(h8, img[m * (8 * B) + L.a_idx]);
        }
        f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 4; ++m) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m], __builtin_bit_cast(h8, b[m]), d, 0, 0, 0);
        const float4 sx = ldsSx[Tl * (HALF / 2) + uint32_t(t0 / 2)];
        acc[0] = __builtin_fmaf(sx.z, d[0], acc[0]);
        acc[1] = __builtin_fmaf(sx.z, d[1], acc[1]);
        acc[2] = __builtin_fmaf(sx.w, d[2], acc[2]);
        acc[3] = __builtin_fmaf(sx.w, d[3], acc[3]);
    };
    for (uint32_t base = 0; base < nE; base += P) {
#pragma unroll
        for (int j = 0; j < P; j += 2) {
            const uint32_t E = base + uint32_t(j);
            if (E < nE) {
                u4 b[4];
                exchange(ring[j], b[0], b[1]);
                exchange(ring[j + 1], b[2], b[3]);
                tile(b, Ta + E / 2u);
            }
            __builtin_amdgcn_sched_barrier(0);
            issue(ring[j], E + P);
            issue(ring[j + 1], E + 1u + P);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- 5. The row's sums (hi + lo, then the tile's runs in order); y, or
    // the split's slots. ----
    float v0 = acc[0] + acc[1], v1 = acc[2] + acc[3];
    if (KW > 1) {
        if (kq > 0) ldsRed[wave * 64u + uint32_t(lane)] = float2{v0, v1};
        lds_barrier();
        if (kq == 0) {
            for (uint32_t k = 1; k < KW; ++k) {
                const float2 o = ldsRed[(wave + k) * 64u + uint32_t(lane)];
                v0 += o.x;
                v1 += o.y;
            }
        }
    }
    const uint32_t row = tile0 + uint32_t(r);
    const bool row_ok = kq == 0 && row < p.rows;
    if (p.ns == 1) {
        if (row_ok) {
            if (t0 < B) p.y[size_t(t0) * p.rows + row] = v0;
            if (t0 + 1 < B) p.y[size_t(t0 + 1) * p.rows + row] = v1;
        }
        return;
    }
    const size_t stride = size_t(B) * p.rows;
    const unsigned long long tag = (unsigned long long)p.epoch << 32;
    unsigned long long *mine = p.slots + size_t(split) * stride;
    if (row_ok) {
        if (t0 < B)
            __hip_atomic_store(mine + size_t(t0) * p.rows + row, tag | __float_as_uint(v0), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if (t0 + 1 < B)
            __hip_atomic_store(mine + size_t(t0 + 1) * p.rows + row, tag | __float_as_uint(v1), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    // The arrival counter only elects the finisher: a slot counts once it
    // carries the launch's epoch, so nothing orders the slot stores against
    // the increments, and every other split incremented after issuing its
    // stores, so the finisher's wait ends as soon as they land.
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&p.counters[band], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = prev + 1 == p.ns;
        if (last) __hip_atomic_store(&p.counters[band], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *ldsLast = last ? 1 : 0;
    }
    __syncthreads();
    if (*ldsLast == 0) return;
    // The finisher: each output's ns slots, requested eight at a time, then
    // taken in split order once tagged.
    bool ok = true;
    const uint32_t band_rows = RT * 16u;
    for (uint32_t i = uint32_t(tid); i < band_rows * B; i += uint32_t(nthr)) {
        const uint32_t t = i / band_rows;
        const uint32_t rr = band_row0 + i % band_rows;
        if (rr >= p.rows) continue;
        unsigned long long *first = p.slots + size_t(t) * p.rows + rr;
        constexpr uint32_t kChunk = 8;
        float sum = 0.f;
        for (uint32_t k0 = 0; k0 < p.ns; k0 += kChunk) {
            unsigned long long w[kChunk];
#pragma unroll
            for (uint32_t k = 0; k < kChunk; ++k)
                w[k] = k0 + k < p.ns
                           ? __hip_atomic_load(first + (k0 + k) * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
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
                sum += __uint_as_float(uint32_t(w[k]));
                if (p.reset_slots) __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        p.y[size_t(t) * p.rows + rr] = sum;
    }
    if (!ok && p.status)
        __hip_atomic_store(p.status, 0xA0000000u | band, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

template <int B, int XI, int P>
hipError_t launch_p(const DenseParams &p, uint32_t threads, size_t lds, hipStream_t stream) {
    auto kernel = dense_mfma_kernel<B, XI, P>;
    if (lds > 65536) {
        const hipError_t e = raise_lds_limit(reinterpret_cast<const void *>(kernel), lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, dim3(p.nbands * p.ns), dim3(threads), lds, stream, p);
    return hipGetLastError();
}

// x items per thread: the compiled counts.
constexpr uint32_t dense_xi(uint32_t xi) { return xi <= 1 ? 1 : xi <= 2 ? 2 : xi <= 4 ? 4 : 8; }

template <int B, int P>
hipError_t launch_xi(const DenseParams &p, uint32_t xi, uint32_t threads, size_t lds, hipStream_t stream) {
    switch (dense_xi(xi)) {
        case 1: return launch_p<B, 1, P>(p, threads, lds, stream);
        case 2: return launch_p<B, 2, P>(p, threads, lds, stream);
        case 4: return launch_p<B, 4, P>(p, threads, lds, stream);
        default: return launch_p<B, 8, P>(p, threads, lds, stream);
    }
}

template <int B>
hipError_t launch_b(const DenseParams &p, const DensePlan &pl, hipStream_t stream) {
    const uint32_t threads = pl.rt * pl.kw * 64;
    return pl.ring == 8 ? launch_xi<B, 8>(p, pl.xi, threads, pl.lds, stream)
                        : launch_xi<B, 4>(p, pl.xi, threads, pl.lds, stream);
}

template <int B, int P>
const void *instance_p(uint32_t xi) {
    switch (dense_xi(xi)) {
        case 1: return reinterpret_cast<const void *>(dense_mfma_kernel<B, 1, P>);
        case 2: return reinterpret_cast<const void *>(dense_mfma_kernel<B, 2, P>);
        case 4: return reinterpret_cast<const void *>(dense_mfma_kernel<B, 4, P>);
        default: return reinterpret_cast<const void *>(dense_mfma_kernel<B, 8, P>);
    }
}

template <int B>
const void *instance_b(uint32_t xi, uint32_t ring) {
    return ring == 8 ? instance_p<B, 8>(xi) : instance_p<B, 4>(xi);
}

const void *instance(uint32_t batch, uint32_t xi, uint32_t ring) {
    switch (batch) {
        case 1: return instance_b<1>(xi, ring);
        case 2: return instance_b<2>(xi, ring);
        case 3: return instance_b<3>(xi, ring);
        case 4: return instance_b<4>(xi, ring);
        default: return nullptr;
    }
}

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

// Estimated time (us) of a plan: a fixed start-up, then the stream of the
// weights and of the x every workgroup stages, slowed by the load
// imbalance of the workgroups over the CUs (a CU streams at about its share
// of HBM bandwidth, so the most loaded CU sets the pace), or one wave's
// chain of ring refills if that is longer, plus the repeated start-up of
// further rounds of resident workgroups and, for split plans, the arrival
// election and the finisher's slot reads.
double dense_cost(double bytes, uint32_t batch, uint32_t nbands, uint32_t kw, uint32_t ns, uint32_t tps,
                  uint32_t ring, uint32_t resident, uint32_t cus) {
    const double wgs = double(nbands) * ns;
    const double per_cu = wgs / cus;
    const double balance = per_cu <= 1.0 ? per_cu : per_cu / std::ceil(per_cu);
    const double x_bytes = wgs * tps * 512.0 * batch;
    const double rounds = std::ceil(wgs / (double(resident) * cus));
    const double chain = std::ceil(2.0 * std::ceil(double(tps) / kw) / ring) * kDenseLatencyUs * rounds;
    const double stream = std::max((bytes + kDenseXCost * x_bytes) / kDenseBytesPerUs / balance, chain);
    const double finish = ns > 1 ? kDenseElectUs + kDenseSlotUs * std::ceil(ns / 8.0) : 0.0;
    return kDenseStartUs + stream + kDenseRoundUs * (rounds - 1.0) + finish;
}

// LDS of a workgroup: x images and factors of tps tiles, the K runs' sums
// and the finisher flag.
size_t dense_lds_bytes(uint32_t tps, uint32_t batch, uint32_t threads) {
    return size_t(tps) * (4 * 4 * 2 * batch * 16 + 4 * 16) + size_t(threads) * 8 + 16;
}

}  // namespace

bool dense_mfma_supported(const uint16_t *w, uint32_t rows, uint32_t cols, uint32_t batch) {
    if (batch < 1 || batch > 4 || rows == 0 || cols == 0 || cols % 32 != 0) return false;
    if ((reinterpret_cast<uintptr_t>(w) & 15) != 0) return false;
    return uint64_t(rows) * cols * 2 < (1ull << 31) && uint64_t(batch) * cols * 4 < (1ull << 31);
}

DensePlan plan_dense_mfma(uint32_t rows, uint32_t cols, uint32_t batch, const DeviceLimits &lim,
                          const DenseForce &force) {
    DensePlan pl;
    const uint32_t row_tiles = (rows + 15) / 16;
    const uint32_t tiles = (cols + kTileK - 1) / kTileK;
    const uint32_t cus = lim.num_cus > 0 ? uint32_t(lim.num_cus) : 256u;
    const double bytes = double(rows) * cols * 2;
    double best = 1e30;
    for (uint32_t ring : {4u, 8u}) {
        if (force.ring && ring != force.ring) continue;
        for (uint32_t rt : {1u, 2u, 4u, 8u}) {
            if (force.rt && rt != force.rt) continue;
            if (rt > row_tiles && rt > 1) continue;
            const uint32_t nbands = (row_tiles + rt - 1) / rt;
            for (uint32_t kw : {1u, 2u, 4u, 8u}) {
                if (force.kw && kw != force.kw) continue;
                if (rt * kw > uint32_t(kMaxWaves)) continue;
                for (uint32_t ns = 1; ns <= tiles && ns <= kMaxDenseSplits; ++ns) {
                    if (force.ns && ns != force.ns) continue;
                    const uint32_t tps = (tiles + ns - 1) / ns;
                    if ((tiles + tps - 1) / tps != ns || kw > tps) continue;
                    const uint32_t threads = rt * kw * 64;
                    const uint32_t xi = (tps * batch * 16 + threads - 1) / threads;
                    if (xi > 8) continue;
                    const size_t lds = dense_lds_bytes(tps, batch, threads);
                    if (lds > lim.max_lds_per_block) continue;
                    const uint32_t resident = resident_per_cu(instance(batch, dense_xi(xi), ring), threads, lds);
                    const double score = dense_cost(bytes, batch, nbands, kw, ns, tps, ring, resident, cus);
                    if (score < best - 1e-9) {
                        best = score;
                        pl.cost_us = score;
                        pl.rt = rt;
                        pl.kw = kw;
                        pl.ring = ring;
                        pl.nbands = nbands;
                        pl.ns = ns;
                        pl.tiles = tiles;
                        pl.tps = tps;
                        pl.xi = xi;
                        pl.lds = lds;
                    }
                }
            }
        }
    }
    if (pl.rt == 0 && (force.rt || force.kw || force.ns || force.ring))
        return plan_dense_mfma(rows, cols, batch, lim, DenseForce{});
    return pl;
}

size_t dense_mfma_workspace(const DensePlan &pl, uint32_t rows, uint32_t batch) {
    return pl.ns > 1 ? size_t(pl.ns) * batch * rows * sizeof(unsigned long long) : 0;
}

hipError_t launch_dense_mfma(const uint16_t *w, const float *x, float *y, uint32_t rows, uint32_t cols,
                             uint32_t batch, const DensePlan &pl, unsigned long long *slots, uint32_t *counters,
                             uint32_t epoch, const TileWait &wait, hipStream_t stream) {
    if (pl.rt == 0 || pl.kw == 0 || pl.rt * pl.kw > uint32_t(kMaxWaves) || (pl.ring != 4 && pl.ring != 8) ||
        !dense_mfma_supported(w, rows, cols, batch))
        return hipErrorInvalidValue;
    if (pl.ns > 1 && (slots == nullptr || counters == nullptr)) return hipErrorInvalidValue;
    DenseParams p;
    p.w = w;
    p.x = x;
    p.y = y;
    p.slots = slots;
    p.counters = counters;
    p.rows = rows;
    p.cols = cols;
    p.w_bytes = uint32_t(uint64_t(rows) * cols * 2);
    p.nbands = pl.nbands;
    p.ns = pl.ns;
    p.tiles = pl.tiles;
    p.tps = pl.tps;
    p.kw = pl.kw;
    p.epoch = epoch;
    p.wait_epoch = wait.force_give_up ? epoch + 0x40000000u : epoch;
    p.spin_limit = wait.force_give_up ? 64u : 1u << 22;
    p.status = wait.status;
    p.reset_slots = wait.reset_slots ? 1u : 0u;
    switch (batch) {
        case 1: return launch_b<1>(p, pl, stream);
        case 2: return launch_b<2>(p, pl, stream);
        case 3: return launch_b<3>(p, pl, stream);
        default: return launch_b<4>(p, pl, stream);
    }
}

}  // namespace qmr

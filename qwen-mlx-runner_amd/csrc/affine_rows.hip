// Streaming dequantise + GEMV / small block (batch 1..4) over MLX affine
// packed weights on the gfx950 matrix cores, with every workgroup owning
// whole rows.
//
// Same product and numerics as affine_mfma.hip (operands, code encoding and
// the tile product are in mfma_common.hpp):
//     y[t*rows + r] = sum_g ( s[r,g] * sum_{c in g} q[r,c] * x[t,c]
//                           + b[r,g] * sum_{c in g} x[t,c] )
// which is the reference's per-weight affine dot (kernels/qwen.metal:40-68,
// kernels/matmul_block.metal:20-79) in the factored form of
// kernels/matvec_fast.metal:11-15.
//
// Decomposition. A workgroup owns RT 16-row tiles for the whole of K and
// runs KW waves per tile; wave (tile, kw) takes the 128-byte entries
// kw, kw + KW, kw + 2KW, ... of its 16 rows, so the workgroup sweeps K in
// chunks of KW*J entries (J per wave).
//   - Staging: per chunk the workgroup stages x (hi/lo MFMA operands, group
//     sums, epilogue factors) and the tiles' metadata in LDS. Two buffers:
//     chunk c+1 is staged while chunk c is multiplied, with one LDS-only
//     barrier per chunk (the weight loads stay in flight across it). The
//     staging loads of chunk c+2 are issued at the end of chunk c, J entries
//     before they are needed, which covers their latency. The RT tiles share
//     the staged x.
//   - Codes: each wave keeps P entries in flight in a register ring. An entry
//     is loaded coalesced (eight consecutive lanes read one row's 128
//     contiguous bytes, rows 0-7 then 8-15) and goes through a per-wave LDS
//     transpose into the MFMA layout (lane (r, g) holds row r's K chunk g).
//     Loading in the MFMA order directly, with consecutive lanes on
//     different rows, streams about 10% slower on this part.
//   - End: the KW partial sums of a row are added in LDS in wave order and
//     written to y. There is no workspace, no atomic and no synchronisation
//     between workgroups, and results do not depend on timing.
// Use: the default where the split-K kernel's per-workgroup costs are not
// amortised (grids past one round of resident workgroups, such as a
// vocabulary head, and splits under four K tiles, such as a Q8 5120x5120
// projection), the fused MLP form (MODE 1 below) always, and the tuning
// hook rr = -3. On the MLP shapes the split-K kernel stays faster (14-15 us
// against 15-16): with rows/16 tiles (320 for 5120 rows) and two entries in
// flight per wave, fewer bytes are in flight to cover HBM latency, and the
// per-chunk staging and tile products sit on each wave's critical path.
//
// Load order per wave: memory counters retire in issue order, so waiting for
// a load also waits for every load issued before it. The staging loads of
// chunk c+2, issued at the end of chunk c after the ring load of entry
// i + P, are waited for at the end of chunk c+1, when that entry (J >= P
// steps later) has already been consumed.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "kernels.hpp"
#include "mfma_common.hpp"

namespace qmr {
namespace {

using namespace mfma;

constexpr int kMaxWaves = 16;
constexpr int kRing = 2;      // entries in flight per wave
constexpr int kXItems = 1;    // staged x slices per thread per chunk
constexpr int kMUnits = 2;    // staged metadata loads per thread per chunk
constexpr int kTPitch = 144;  // bytes per row of a wave's transpose scratch (128 + pad)

struct RowsParams {
    const uint32_t *w;
    const void *s;
    const void *b;
    const float *x;
    float *y;
    uint32_t rows, cols;
    uint32_t w_bytes, m_bytes;  // extents of the code and metadata views
    uint32_t rt, kw;            // row tiles and K waves per workgroup
    uint32_t j;                 // entries per wave per chunk
    uint32_t n_entries;         // 128-byte entries per row (the last may be partial)
    uint32_t n_chunks;          // ceil(n_entries / (kw * j))
    uint32_t stage_bytes;       // one LDS staging buffer (16-byte multiple)
    // Fused forms (AffineArgs): the residual added to y, and for the MLP form
    // the up matrix, the RMS-norm weights and epsilon.
    const float *r;
    const uint32_t *w2;
    const void *s2;
    const void *b2;
    const float *norm;
    float eps;
};

// MODE 0: y = W x (+ residual). MODE 1, the MLP form: the first rt/2 row
// tiles of a workgroup are gate rows and the last rt/2 the up rows with the
// same indices, x is staged as x * norm (the RMS norm's weights; its 1/rms
// factor is applied to the sums), and y = silu(gate) * up.
template <int BITS, int META, int GROUP, int B, bool PAIRS, int MODE>
__global__ __launch_bounds__(kMaxWaves * 64) void affine_rows_kernel(RowsParams p) {
    constexpr int NGM = kTileK / GROUP;  // quant groups per tile
    constexpr int SLOTS = 16 / NGM;      // A rows per quant group
    constexpr int HALF = SLOTS / 2;      // RHS per quant group in D (>= B)
    constexpr int NLD = BITS / 4;        // 16-byte code pieces per lane per tile
    constexpr int MB = META == 0 ? 4 : 2;
    constexpr int MW = META == 0 ? 2 : 1;  // LDS words per metadata entry
    constexpr int UE = PAIRS ? 2 : 1;      // entries per staged metadata load
    constexpr int TPE = 8 / BITS;          // K tiles per 128-byte entry
    constexpr int P = kRing;
    static_assert(2 * B <= SLOTS, "batch does not fit the slot layout");
    static_assert(!PAIRS || MB == 2, "paired metadata loads need 16-bit entries");

    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int r = lane & 15;
    const int lg = lane >> 4;
    const uint32_t KW = p.kw;
    const uint32_t ti = uint32_t(wave) / KW;
    const uint32_t kw = uint32_t(wave) - ti * KW;
    const uint32_t J = p.j;
    const uint32_t CT = KW * J * TPE;        // K tiles per chunk
    const uint32_t gpc = CT * NGM;           // quant groups per chunk
    const uint32_t Gp = gpc | 1;             // LDS pitch of a row's staged metadata (odd)
    constexpr bool MLP = MODE == 1;
    const uint32_t RTH = MLP ? p.rt / 2 : p.rt;  // row tiles per matrix
    const uint32_t mat = MLP ? uint32_t(__builtin_amdgcn_readfirstlane(int(ti >= RTH))) : 0u;
    const uint32_t row0 = blockIdx.x * RTH * 16;
    const uint32_t tile0 = row0 + (ti - mat * RTH) * 16;

    // LDS: [staging buffer 0][staging buffer 1][transpose scratch per wave][sums]
    // A staging buffer: A operands [CT][4 m][4 g][2B] u4, Sx [CT][NGM][HALF/2]
    // float4, metadata [RT*16 rows][Gp] entries.
    const size_t sx_off = size_t(CT) * 4 * 4 * 2 * B * 16;
    const size_t m_off = sx_off + size_t(CT) * NGM * (HALF / 2) * 16;
    auto stage_ptr = [&](uint32_t buf) { return lds + size_t(buf) * p.stage_bytes; };
    unsigned char *trans = lds + 2 * size_t(p.stage_bytes);
    unsigned char *tw = trans + size_t(wave) * 16 * kTPitch;
    float *red = reinterpret_cast<float *>(trans + size_t(nthr / 64) * 16 * kTPitch);

    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t *>(mat ? p.w2 : p.w), 0, int(p.w_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.s), 0, int(p.m_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t br =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.b), 0, int(p.m_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(p.x), 0, int(uint32_t(B) * p.cols * 4u), kRsrcWord3);
    // MLP form only (the pointers are null otherwise and these go unused).
    const __amdgpu_buffer_rsrc_t sr2 =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.s2), 0, int(p.m_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t br2 =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.b2), 0, int(p.m_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t nr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p.norm), 0, int(p.cols * 4u), kRsrcWord3);

    // ---- Staging of one chunk: loads into registers, then conversion into
    // an LDS buffer. Loads are issued only by waves with work (a wave-uniform
    // test); groups past the row end and columns past cols read as zeros. ----
    const uint32_t m_pitch = p.cols / GROUP;
    const uint32_t upr = (gpc + UE - 1) / UE;  // metadata loads per row per chunk
    const uint32_t units = p.rt * 16 * upr;
    const uint32_t items = CT * B * 16;
    const uint32_t wave_base = __builtin_amdgcn_readfirstlane(uint32_t(tid) & ~63u);
    float xv[kXItems][8];
    uint32_t mv_s[kMUnits], mv_b[kMUnits];
    auto stage_load = [&](uint32_t c) {
#pragma unroll
        for (int i = 0; i < kXItems; ++i) {
#pragma unroll
            for (int j = 0; j < 8; ++j) xv[i][j] = 0.f;
            if (wave_base + i * nthr >= items) continue;
            const uint32_t it = tid + i * nthr;
            load_x8(xv[i], xr, uint32_t(item_pos<B>(it).t), c * CT * kTileK + item_col<B>(it), p.cols,
                    it < items);
            if constexpr (MLP) {
                float nv[8];
                load_x8(nv, nr, 0u, c * CT * kTileK + item_col<B>(it), p.cols, it < items);
#pragma unroll
                for (int j = 0; j < 8; ++j) xv[i][j] *= nv[j];
            }
        }
#pragma unroll
        for (int u = 0; u < kMUnits; ++u) {
            mv_s[u] = mv_b[u] = 0u;
            if (wave_base + u * nthr >= units) continue;
            const uint32_t f = tid + u * nthr;
            const uint32_t rl = f / upr;
            const uint32_t g = c * gpc + (f - rl * upr) * UE;
            // MLP form: staged rows RTH*16.. are the up matrix's rows 0...
            const bool second = MLP && rl >= RTH * 16;
            const uint32_t mrow = row0 + rl - (second ? RTH * 16 : 0u);
            const uint32_t off = (f < units && g < m_pitch) ? (mrow * m_pitch + g) * MB : kOut;
            const uint32_t off1 = second ? kOut : off;
            if constexpr (MB == 4 || PAIRS) {
                mv_s[u] = __builtin_amdgcn_raw_buffer_load_b32(sr, int(off1), 0, 0);
                mv_b[u] = __builtin_amdgcn_raw_buffer_load_b32(br, int(off1), 0, 0);
                if constexpr (MLP) {
                    const uint32_t off2 = second ? off : kOut;
                    mv_s[u] |= __builtin_amdgcn_raw_buffer_load_b32(sr2, int(off2), 0, 0);
                    mv_b[u] |= __builtin_amdgcn_raw_buffer_load_b32(br2, int(off2), 0, 0);
                }
            } else {
                mv_s[u] = __builtin_amdgcn_raw_buffer_load_b16(sr, int(off1), 0, 0);
                mv_b[u] = __builtin_amdgcn_raw_buffer_load_b16(br, int(off1), 0, 0);
                if constexpr (MLP) {
                    const uint32_t off2 = second ? off : kOut;
                    mv_s[u] |= __builtin_amdgcn_raw_buffer_load_b16(sr2, int(off2), 0, 0);
                    mv_b[u] |= __builtin_amdgcn_raw_buffer_load_b16(br2, int(off2), 0, 0);
                }
            }
        }
    };
    auto stage_store = [&](uint32_t buf) {
        unsigned char *sp = stage_ptr(buf);
        uint32_t *M = reinterpret_cast<uint32_t *>(sp + m_off);
#pragma unroll
        for (int u = 0; u < kMUnits; ++u) {
            const uint32_t f = tid + u * nthr;
            if (f < units) {
                const uint32_t rl = f / upr;
                uint32_t *dst = M + (rl * Gp + (f - rl * upr) * UE) * MW;
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
        u4 *A = reinterpret_cast<u4 *>(sp);
        float4 *Sx = reinterpret_cast<float4 *>(sp + sx_off);
#pragma unroll
        for (int i = 0; i < kXItems; ++i) {
            const uint32_t it = tid + i * nthr;
            if (i > 0 && it >= items) break;  // whole 16-lane blocks are in or out
            stage_x_item<BITS, GROUP, B>(xv[i], it, it < items, lane, A, Sx);
        }
        stage_x_pads<GROUP, B>(CT, tid, nthr, Sx);
    };

    // ---- Weight entries: coalesced loads (lane -> row lane/8 of the half,
    // 16-byte piece lane%8); bytes past the row end read as zeros. ----
    const uint32_t row_bytes = p.cols / 32 * (BITS * 4);
    const uint32_t lrow = uint32_t(lane) >> 3;
    const uint32_t piece = uint32_t(lane) & 7;
    const uint32_t base1 = (tile0 + lrow) * row_bytes + 16 * piece;
    const uint32_t base2 = base1 + 8 * row_bytes;
    auto issue = [&](u4 (&c)[2], uint32_t i) {
        const uint32_t eb = (kw + KW * i) * 128;
        const bool ok = eb + 16 * piece < row_bytes;
        c[0] = __builtin_amdgcn_raw_buffer_load_b128(wr, int(ok ? base1 + eb : kOut), 0, kAuxStream);
        c[1] = __builtin_amdgcn_raw_buffer_load_b128(wr, int(ok ? base2 + eb : kOut), 0, kAuxStream);
    };
    // Transpose through this wave's scratch: afterwards `kept` and `got` are
    // the pieces kp and sp of row r (Q4: tile 0 and tile 1 of the entry; Q8:
    // the two halves of the lane's 32-byte chunk).
    const uint32_t kp = BITS == 4 ? uint32_t(lg) : 2u * lg;
    const uint32_t sp = BITS == 4 ? uint32_t(lg) + 4 : 2u * lg + 1;
    unsigned char *tw_lane = tw + lrow * kTPitch + 16 * piece;
    const unsigned char *tr_lane = tw + uint32_t(r) * kTPitch;
    auto transpose_write = [&](const u4 (&c)[2]) {
        *reinterpret_cast<u4 *>(tw_lane) = c[0];
        *reinterpret_cast<u4 *>(tw_lane + 8 * kTPitch) = c[1];
        wave_lds_sync();
    };
    auto transpose_read = [&](u4 &kept, u4 &got) {
        kept = *reinterpret_cast<const u4 *>(tr_lane + 16 * kp);
        got = *reinterpret_cast<const u4 *>(tr_lane + 16 * sp);
        wave_lds_sync();
    };

    const LaneMap<GROUP, B> L(lane);
    const uint32_t m_idx = (ti * 16 + uint32_t(r)) * Gp + uint32_t(L.gD);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    h8 a[4] = {h8{}, h8{}, h8{}, h8{}};
    auto compute = [&](const u4 (&c)[NLD], uint32_t buf, uint32_t Tl) {
        const unsigned char *sp_ = stage_ptr(buf);
        const u4 *A = reinterpret_cast<const u4 *>(sp_);
        const float4 *Sx = reinterpret_cast<const float4 *>(sp_ + sx_off);
        const uint32_t *M = reinterpret_cast<const uint32_t *>(sp_ + m_off);
        float sv, bv;
        meta_entry<META>(M + (m_idx + Tl * NGM) * MW, sv, bv);
        const float4 sx = Sx[(Tl * NGM + L.gD) * (HALF / 2) + L.t0 / 2];
        tile_product<BITS, META, GROUP, B>(c, L, A + Tl * 4 * (8 * B), sv, bv, sx, a, acc);
    };

    // ---- Prologue: stage chunk 0, request the first P entries, load the
    // staging of chunk 1. ----
    stage_load(0);
    u4 ring[P][2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < P; ++j) {
        issue(ring[j], uint32_t(j));
        __builtin_amdgcn_sched_barrier(0);
    }
    // MLP form: sum of squares of each x[t] (the RMS norm's statistic),
    // reduced per wave into the sums area (unused until the epilogue), while
    // the first weight entries are in flight.
    if constexpr (MLP) {
        float sq[B];
#pragma unroll
        for (int t = 0; t < B; ++t) {
            sq[t] = 0.f;
            for (uint32_t k = uint32_t(tid) * 4u; k < p.cols; k += uint32_t(nthr) * 4u) {
                const u4 v = __builtin_amdgcn_raw_buffer_load_b128(xr, int((uint32_t(t) * p.cols + k) * 4u), 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e) sq[t] += __uint_as_float(v[e]) * __uint_as_float(v[e]);
            }
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) sq[t] += __shfl_xor(sq[t], m, 64);
            if (lane == 0) red[wave * B + t] = sq[t];
        }
    }
    stage_store(0);
    if (p.n_chunks > 1) stage_load(1);
    lds_barrier();
    // 1/rms of this lane's RHS in the epilogue (lane/16), from the per-wave sums.
    float inv_t = 1.f;
    if constexpr (MLP) {
        const int t = (lane >> 4) < B ? (lane >> 4) : 0;
        float ss = 0.f;
        for (int wv = 0; wv < nthr / 64; ++wv) ss += red[wv * B + t];
        inv_t = 1.0f / sqrtf(ss / float(p.cols) + p.eps);
    }

    // ---- This wave's entries i = 0, 1, ... (entry kw + KW*i, chunk i / J).
    // Every wave runs the same number of steps, so the barriers match. ----
    const uint32_t steps = p.n_chunks * J;
    uint32_t c = 0, jj = 0;  // chunk of step i and its position in the chunk
    for (uint32_t i0 = 0; i0 < steps; i0 += P) {
#pragma unroll
        for (int j = 0; j < P; ++j) {
            const uint32_t i = i0 + j;
            if (i < steps) {
                // The ring slot is free once its entry is in the transpose
                // scratch: request entry i + P before multiplying entry i.
                const bool live = (kw + KW * i) * 128 < row_bytes;
                if (live) transpose_write(ring[j]);
                __builtin_amdgcn_sched_barrier(0);
                issue(ring[j], i + P);
                __builtin_amdgcn_sched_barrier(0);
                if (live) {
                    u4 kept, got;
                    transpose_read(kept, got);
                    const uint32_t Tl = (kw + KW * jj) * TPE;  // tile within the chunk
                    if constexpr (BITS == 4) {
                        const u4 c0v[1] = {kept};
                        const u4 c1v[1] = {got};
                        compute(c0v, c & 1, Tl);
                        compute(c1v, c & 1, Tl + 1);
                    } else {
                        const u4 cv[2] = {kept, got};
                        compute(cv, c & 1, Tl);
                    }
                }
                const bool chunk_end = jj + 1 == J;
                if (chunk_end && c + 1 < p.n_chunks) {
                    stage_store((c + 1) & 1);
                    if (c + 2 < p.n_chunks) stage_load(c + 2);
                }
                if (chunk_end) {
                    lds_barrier();
                    ++c;
                    jj = 0;
                } else {
                    ++jj;
                }
            }
        }
    }

    // ---- The KW partial sums of each row, added in wave order. ----
    float v0, v1;
    combine_slots<GROUP>(acc, v0, v1);
    float *rw = red + (size_t(ti) * KW + kw) * (B * 16);
    if (lg < 4 / NGM) {
        if (L.t0 < B) rw[L.t0 * 16 + r] = v0;
        if (L.t0 + 1 < B) rw[(L.t0 + 1) * 16 + r] = v1;
    }
    __syncthreads();
    if (kw == 0 && lane < B * 16 && (!MLP || ti < RTH)) {
        const int t = lane >> 4;
        const uint32_t row = tile0 + uint32_t(lane & 15);
        float sum = 0.f;
        for (uint32_t k = 0; k < KW; ++k) sum += red[((ti * KW + k) * B + t) * 16 + (lane & 15)];
        if constexpr (MLP) {
            // The up rows with the same indices sit in tile ti + RTH.
            float up = 0.f;
            for (uint32_t k = 0; k < KW; ++k) up += red[(((ti + RTH) * KW + k) * B + t) * 16 + (lane & 15)];
            const float g = sum * inv_t;
            sum = g * (1.0f / (1.0f + expf(-g))) * (up * inv_t);
        }
        if (row < p.rows) {
            const size_t o = size_t(t) * p.rows + row;
            p.y[o] = p.r ? p.r[o] + sum : sum;
        }
    }
}

template <int BITS, int META, int GROUP, int B, bool PAIRS>
hipError_t launch_b(const RowsParams &p, uint32_t nbands, size_t lds, hipStream_t stream) {
    auto kernel = p.w2 ? affine_rows_kernel<BITS, META, GROUP, B, PAIRS, 1>
                       : affine_rows_kernel<BITS, META, GROUP, B, PAIRS, 0>;
    if (lds > 65536) {
        const hipError_t e = raise_lds_limit(reinterpret_cast<const void *>(kernel), lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, dim3(nbands), dim3(p.rt * p.kw * 64), lds, stream, p);
    return hipGetLastError();
}

template <int BITS, int META, int GROUP, int B>
hipError_t launch_pairs(const RowsParams &p, bool pairs, uint32_t nbands, size_t lds, hipStream_t stream) {
    if constexpr (META != 0) {
        if (pairs) return launch_b<BITS, META, GROUP, B, true>(p, nbands, lds, stream);
    }
    return launch_b<BITS, META, GROUP, B, false>(p, nbands, lds, stream);
}

template <int BITS, int META, int GROUP>
hipError_t launch_group(const RowsParams &p, uint32_t batch, bool pairs, uint32_t nbands, size_t lds,
                        hipStream_t stream) {
    constexpr int MAXB = (16 / (kTileK / GROUP)) / 2;
    switch (batch) {
        case 1: return launch_pairs<BITS, META, GROUP, 1>(p, pairs, nbands, lds, stream);
        case 2: return launch_pairs<BITS, META, GROUP, 2>(p, pairs, nbands, lds, stream);
        case 3:
            if constexpr (MAXB >= 3) return launch_pairs<BITS, META, GROUP, 3>(p, pairs, nbands, lds, stream);
            break;
        case 4:
            if constexpr (MAXB >= 4) return launch_pairs<BITS, META, GROUP, 4>(p, pairs, nbands, lds, stream);
            break;
        default: break;
    }
    return hipErrorInvalidValue;
}

template <int BITS, int META>
hipError_t launch_meta(const RowsParams &p, uint32_t group, uint32_t batch, bool pairs, uint32_t nbands,
                       size_t lds, hipStream_t stream) {
    switch (group) {
        case 32: return launch_group<BITS, META, 32>(p, batch, pairs, nbands, lds, stream);
        case 64: return launch_group<BITS, META, 64>(p, batch, pairs, nbands, lds, stream);
        case 128: return launch_group<BITS, META, 128>(p, batch, pairs, nbands, lds, stream);
        default: return hipErrorInvalidValue;
    }
}

size_t rows_stage_bytes(uint32_t kw, uint32_t j, uint32_t rt, uint32_t bits, uint32_t group,
                        uint32_t batch, bool f32_meta) {
    const uint32_t ct = kw * j * (8 / bits);
    const uint32_t ngm = kTileK / group;
    const uint32_t half = 16 / ngm / 2;
    const size_t gp = (size_t(ct) * ngm) | 1;
    const size_t bytes = size_t(ct) * 4 * 4 * 2 * batch * 16 + size_t(ct) * ngm * (half / 2) * 16 +
                         size_t(rt) * 16 * gp * 4 * (f32_meta ? 2 : 1);
    return (bytes + 15) / 16 * 16;
}

size_t rows_lds_bytes(uint32_t kw, uint32_t j, uint32_t rt, uint32_t bits, uint32_t group,
                      uint32_t batch, bool f32_meta) {
    return 2 * rows_stage_bytes(kw, j, rt, bits, group, batch, f32_meta) + size_t(rt) * kw * 16 * kTPitch +
           size_t(rt) * kw * batch * 16 * 4;
}

}  // namespace

bool affine_rows_supported(const AffineArgs &a) { return affine_mfma_supported(a); }

namespace {

// The tiling search behind plan_affine_rows and plan_affine_mlp. The MLP form
// stacks the gate and up tiles of the same rows: twice the row tiles, rt even.
RowsPlan plan_rows(const AffineArgs &a, const DeviceLimits &lim, uint32_t force_rt, uint32_t force_kw,
                   uint32_t force_j, bool mlp) {
    RowsPlan best;
    if (!affine_rows_supported(a)) return best;
    const uint32_t row_tiles = (a.rows + 15) / 16 * (mlp ? 2 : 1);
    const uint32_t row_bytes = a.cols / 32 * (a.bits * 4);
    const uint32_t n_entries = (row_bytes + 127) / 128;
    const uint32_t ngm = kTileK / a.group;
    const uint32_t m_pitch = a.cols / a.group;
    const uint32_t tpe = 8 / a.bits;
    const bool f32_meta = a.meta == Meta::F32;
    const double cus = lim.num_cus > 0 ? double(lim.num_cus) : 256.0;
    double best_score = 1e30;
    for (uint32_t rt = 1; rt <= 8; rt *= 2) {
        for (uint32_t kw = 1; kw <= 16; kw *= 2) {
            if (rt * kw > uint32_t(kMaxWaves) || rt * kw < 2 || (mlp && rt < 2)) continue;
            if (force_rt && (rt != force_rt || kw != force_kw)) continue;
            const uint32_t threads = 64 * rt * kw;
            const uint32_t per_wave = (n_entries + kw - 1) / kw;
            for (uint32_t j = 1; j <= 8; j *= 2) {
                if (force_j ? j != force_j : (j > 1 && j > per_wave)) continue;
                // Per-thread staging capacity: x slices and metadata loads of a chunk.
                const uint32_t gpc = kw * j * tpe * ngm;
                const bool pairs = !f32_meta && m_pitch % 2 == 0 && gpc % 2 == 0;
                if (kw * j * tpe * a.batch * 16 > uint32_t(kXItems) * threads) continue;
                if (rt * 16 * ((gpc + (pairs ? 1 : 0)) / (pairs ? 2 : 1)) > uint32_t(kMUnits) * threads) continue;
                const size_t lds = rows_lds_bytes(kw, j, rt, a.bits, a.group, a.batch, f32_meta);
                if (lds > lim.max_lds_per_block) continue;
                const uint32_t nbands = (row_tiles + rt - 1) / rt;
                const uint32_t n_chunks = (n_entries + kw * j - 1) / (kw * j);
                // Score: about eight waves per CU, workgroups of about sixteen
                // waves (more bytes requested per workgroup), at least one
                // workgroup per CU, few idle steps (a partial last chunk),
                // staging requested several entries ahead (J), and staged x
                // shared by several tiles when the block is wide. The weights
                // were fitted to MI355X timings of every (rt, kw, j) on Q4
                // and Q8 matrices from 2048x2048 to the 151936x5120 head.
                const double waves = double(nbands) * rt * kw;
                const double fill = double(n_entries) / (double(n_chunks) * kw * j);
                double score = std::fabs(std::log2(waves / (8.0 * cus))) + 1.0 * (1.0 - fill) +
                               0.25 * a.batch / rt + 0.5 * (j >= 4 ? 0.0 : j == 2 ? 0.5 : 1.0) +
                               0.25 * std::fabs(std::log2(double(rt * kw) / 16.0));
                if (nbands < cus) score += 0.5 * std::log2(cus / nbands);
                // MLP form: two gate and two up tiles per workgroup measured
                // best (17408x5120 at B=1: 29.4 us against 32.5 with eight).
                if (mlp) score += 0.5 * std::fabs(std::log2(double(rt) / 4.0));
                if (row_tiles % rt) score += 1.0 - double(row_tiles) / (double(nbands) * rt);
                if (score < best_score - 1e-9) {
                    best_score = score;
                    best.rt = rt;
                    best.kw = kw;
                    best.j = j;
                    best.nbands = nbands;
                    best.n_entries = n_entries;
                    best.n_chunks = n_chunks;
                    best.pairs = pairs;
                    best.stage_bytes = rows_stage_bytes(kw, j, rt, a.bits, a.group, a.batch, f32_meta);
                    best.lds = lds;
                }
            }
        }
    }
    return best;
}

}  // namespace

RowsPlan plan_affine_rows(const AffineArgs &a, const DeviceLimits &lim, uint32_t force_rt, uint32_t force_kw,
                          uint32_t force_j) {
    return plan_rows(a, lim, force_rt, force_kw, force_j, false);
}

RowsPlan plan_affine_mlp(const AffineArgs &a, const DeviceLimits &lim, uint32_t force_rt, uint32_t force_kw,
                         uint32_t force_j) {
    return plan_rows(a, lim, force_rt, force_kw, force_j, true);
}

hipError_t launch_affine_rows(const AffineArgs &a, const RowsPlan &pl, hipStream_t stream) {
    if (pl.rt == 0) return hipErrorInvalidValue;
    RowsParams p;
    p.w = a.w;
    p.s = a.s;
    p.b = a.b;
    p.x = a.x;
    p.y = a.y;
    p.rows = a.rows;
    p.cols = a.cols;
    p.w_bytes = uint32_t(uint64_t(a.rows) * a.cols * a.bits / 8);
    p.m_bytes = uint32_t(uint64_t(a.rows) * (a.cols / a.group) * (a.meta == Meta::F32 ? 4 : 2));
    p.rt = pl.rt;
    p.kw = pl.kw;
    p.j = pl.j;
    p.n_entries = pl.n_entries;
    p.n_chunks = pl.n_chunks;
    p.stage_bytes = uint32_t(pl.stage_bytes);
    p.r = a.residual;
    p.w2 = a.up_w;
    p.s2 = a.up_s;
    p.b2 = a.up_b;
    p.norm = a.norm;
    p.eps = a.eps;
    if (a.up_w && (pl.rt % 2 != 0 || !a.up_s || !a.up_b || !a.norm)) return hipErrorInvalidValue;
    const int meta = static_cast<int>(a.meta);
    if (a.bits == 4) {
        if (meta == 0) return launch_meta<4, 0>(p, a.group, a.batch, false, pl.nbands, pl.lds, stream);
        if (meta == 1) return launch_meta<4, 1>(p, a.group, a.batch, pl.pairs, pl.nbands, pl.lds, stream);
        return launch_meta<4, 2>(p, a.group, a.batch, pl.pairs, pl.nbands, pl.lds, stream);
    }
    if (meta == 0) return launch_meta<8, 0>(p, a.group, a.batch, false, pl.nbands, pl.lds, stream);
    if (meta == 1) return launch_meta<8, 1>(p, a.group, a.batch, pl.pairs, pl.nbands, pl.lds, stream);
    return launch_meta<8, 2>(p, a.group, a.batch, pl.pairs, pl.nbands, pl.lds, stream);
}

}  // namespace qmr

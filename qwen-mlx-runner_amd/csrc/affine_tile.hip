// Streaming dequantise + GEMV / small block (batch 1..4) over MLX affine
// packed weights on the gfx950 matrix cores: row bands of 16-row tiles, each
// band's K range cut into at most a few long splits across workgroups and
// into contiguous per-wave ranges inside a workgroup.
//
// Same product and numerics as affine_mfma.hip (operands, code encoding and
// the tile product are in mfma_common.hpp):
//     y[t*rows + r] = sum_g ( s[r,g] * sum_{c in g} q[r,c] * x[t,c]
//                           + b[r,g] * sum_{c in g} x[t,c] )
// which is the reference's per-weight affine dot (kernels/qwen.metal:40-68,
// kernels/matmul_block.metal:20-79) in the factored form of
// kernels/matvec_fast.metal:11-15.
//
// Decomposition. Workgroup (band, split) owns TR 16-row tiles over the
// split's K range and runs KW waves per tile; wave (tile, kw) streams the
// contiguous run kw of the split's 128-byte entries for its 16 rows. Grid =
// nbands x ns, blockIdx = band + nbands * split.
//
// Why this shape (measured on MI355X with pure-read kernels of the same
// bytes, back-to-back launches over rotating copies):
//   - The order of a tile's loads costs little (16-byte loads in MFMA lane
//     order read ~14% slower than eight lanes per 128-byte line).
//   - x is read from L2 by every workgroup that needs it, and that traffic
//     competes with the weight stream: one 16-byte x load per lane per entry
//     interleaved with the stream added ~20% at 5120x17408 for 16-row
//     workgroups. So x is staged once per workgroup, up front, shared by all
//     TR*16 rows, and converted there into MFMA operand images in LDS.
//   - A CU streams at most ~45 GB/s here, so a grid needs more than ~160
//     busy CUs: tall bands are cut into a few K splits rather than made
//     into fewer workgroups.
//   - Metadata read as the 32-byte pieces of short splits cost ~20%; long
//     splits read each row's metadata as one run, staged in LDS up front.
// End of a band. The KW partial sums of a row are added in LDS in wave order.
// With ns > 1 splits, splits 0..ns-2 publish their sums as 64-bit slots
// {value, launch epoch} and the band's last split (the highest workgroup
// index, dispatched last) reads them; a slot whose epoch is the current
// launch's is complete, so one read both checks and fetches it, with no
// counter and no fence chain. The sum is taken in split order, so results
// do not depend on timing. The wait is bounded: past the host's spin limit
// the workgroup writes NaN and exits, so every wave always finishes. The
// planner takes split plans only when all their workgroups are resident at
// once; single-split plans, in which no workgroup waits, may span several
// rounds (matrices too tall for one).
//
// Build. This file is compiled once per weight format with
// -DQMR_BAND_BITS=<4|8> -DQMR_BAND_META=<0|1|2>: each such object holds the
// kernel instances of that format (launch_meta, instance_meta), and the
// objects compile in parallel. Compiled without them it holds the planner
// and the launch entry, which call those two through their declarations.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <mutex>
#include <type_traits>
#include <vector>

#include "kernels.hpp"
#include "mfma_common.hpp"

namespace qmr {
namespace band {

constexpr int kMaxThreads = 512;  // up to 8 waves: x staging needs up to 8 items of registers per thread
constexpr uint32_t kBandSplits = 8;    // most K splits of a band
constexpr uint32_t kPlannedSplits = 4; // most the planner picks by itself (more when forced)
constexpr uint32_t kFetchChunk = 4;    // slot words a finisher requests at once, per plane

struct BandParams {
    const uint32_t *w;
    const void *s;
    const void *b;
    const float *x;
    float *y;
    const float *r;              // residual added in the final store (may alias y), or null
    // Fused MLP form: the up matrix (same shape and format as w/s/b, the
    // gate), the RMS-norm weights [cols] and epsilon.
    const uint32_t *w2;
    const void *s2;
    const void *b2;
    const float *norm;
    float eps;
    unsigned long long *partial;  // {value, epoch} slots: [ns-1][B][rows]; MLP form [ns-1][gate, up][B][rows], then [ns-1][nbands][B] sums of x^2
    uint32_t epoch;       // tag of this launch's published sums
    uint32_t wait_epoch;  // tag the last split waits for (the epoch; another value forces the give-up, for tests)
    uint32_t spin_limit;
    uint32_t *status;     // set to 0x80000000 | band by a last split that gives up (may be null)
    uint32_t reset_slots; // nonzero: the finisher clears each slot it took (plain and residual forms)
    uint32_t elect;       // nonzero: every split publishes and an arrival counter elects the finisher
    uint32_t *counters;   // [nbands] arrival counters when elected (zero between launches)
    uint32_t rows, cols;
    uint32_t w_bytes, m_bytes;  // extents of the code and metadata views
    uint32_t tr, kw, ns, nbands;
    uint32_t n_entries;   // 128-byte code entries per row (the last may be partial)
    uint32_t tiles;       // 128-column K tiles
    uint32_t gp;          // LDS pitch of a row's staged metadata (odd)
    uint32_t meta_bytes;  // LDS bytes of the staged metadata (16-byte multiple)
    uint32_t img_bytes;   // LDS bytes of the staged x images
    uint32_t split_e[kBandSplits + 1];  // first entry of each split, then n_entries (host_split_begin)
    uint32_t kw_shift;    // log2(kw)
    uint32_t unit_shift;  // log2 of the threads per row in the metadata loads (>= units per row)
    // Two-phase x staging (single-split plans with one wave per tile): the
    // images of the K tiles [0, phase_tiles) are staged first and those of
    // [phase_tiles, tiles) replace them once every wave has consumed entry
    // phase_entry - 1, so a workgroup holds half the images in LDS.
    uint32_t phase_entry, phase_tiles;
};

// Launches the plan's instance of format <BITS, META> (META 0 f32, 1 bf16,
// 2 f16 scales and biases) for a group size and batch.
template <int BITS, int META>
hipError_t launch_meta(const BandParams &p, const TilePlan &pl, uint32_t group, uint32_t batch, hipStream_t stream);

// The kernel instance for a format, x-item count, ring depth, form (plain
// or the MLP form; the residual form's resources are the plain's) and x
// staging phases (1, or 2 for the plain form), for occupancy queries; null
// for a batch the group size does not allow.
template <int BITS, int META>
const void *instance_meta(uint32_t group, uint32_t batch, uint32_t xi, uint32_t ring, bool mlp, uint32_t phases);

}  // namespace band

#ifdef QMR_BAND_BITS
namespace {

using namespace mfma;
using band::BandParams;
using band::kBandSplits;
using band::kFetchChunk;
using band::kMaxThreads;

constexpr int kMetaUnits = 4;  // 16-byte metadata loads per thread and plane (fast path)

// XI: x items (8 columns each) staged per thread. FUSE 0: y = W x; 1: y =
// r + W x; 2: the fused MLP form, y = silu(G x^) * (U x^) with x^ =
// rms_norm(x) * norm: a band's first TR/2 tiles are gate rows and its last
// TR/2 the up rows with the same indices, so x (staged times the norm
// weights) serves both; the band's last split adds each row's gate and up
// sums in split order and applies 1/rms (the products are linear in it) and
// SwiGLU.
// PH = 2: the two-phase x staging of BandParams (plain and residual forms,
// plans of one split and one wave per tile, so every wave streams the same
// entries and meets the phase barriers together).
template <int BITS, int META, int GROUP, int B, int XI, int P, int FUSE, int PH>
__global__ __launch_bounds__(kMaxThreads) void affine_band_kernel(BandParams p) {
    constexpr bool MLP = FUSE == 2;
    static_assert(PH == 1 || PH == 2, "one or two phases of x staging");
    constexpr int NGM = kTileK / GROUP;  // quant groups per tile
    constexpr int SLOTS = 16 / NGM;      // A rows per quant group
    constexpr int HALF = SLOTS / 2;      // RHS per quant group in D (>= B)
    constexpr int NLD = BITS / 4;        // 16-byte code pieces per lane per tile
    constexpr int TPE = 8 / BITS;        // K tiles per 128-byte entry
    constexpr int MB = META == 0 ? 4 : 2;
    constexpr int VEC = 16 / MB;  // metadata values per 16-byte load
    constexpr uint32_t TIMG_A = 4u * 4 * 2 * B * 16;
    static_assert(2 * B <= SLOTS, "batch does not fit the slot layout");

    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: entry bounds are scalar
    const int lane = tid & 63;
    const int r = lane & 15;
    const int lg = lane >> 4;
    const uint32_t KW = p.kw;
    const uint32_t ti = uint32_t(wave) >> p.kw_shift;
    const uint32_t kw = uint32_t(wave) & (KW - 1u);
    const uint32_t band = blockIdx.x % p.nbands;
    const uint32_t split = blockIdx.x / p.nbands;
    // The MLP form: tiles [0, H) of a band are gate rows, [H, 2H) the up
    // matrix's rows with the same indices; the band's last split finishes.
    const uint32_t H = MLP ? p.tr / 2u : p.tr;  // row tiles per matrix in a band
    const bool up_tile = MLP && ti >= H;        // wave-uniform
    const bool finisher = MLP && split + 1 == p.ns;
    const uint32_t band_row0 = band * H * 16u;
    const uint32_t tile_row0 = band_row0 + (up_tile ? ti - H : ti) * 16u;
    const uint32_t nG = p.cols / GROUP;
    const uint32_t Gp = p.gp;
    // The split's entries (from the host: a uniform select, no division),
    // tiles, groups and columns.
    auto split_at = [&](uint32_t k) -> uint32_t { return p.split_e[k]; };
    const uint32_t SE0 = split_at(split);
    const uint32_t SE1 = split_at(split + 1);
    const uint32_t ST0 = SE0 * TPE;
    const uint32_t ST1 = min(SE1 * TPE, p.tiles);
    const uint32_t nT = ST1 - ST0;
    const uint32_t G0 = ST0 * NGM;
    const uint32_t G1 = min(ST1 * NGM, nG);
    // This wave's entries. The bounds are wave-uniform; readfirstlane keeps
    // them in scalar registers whatever the compiler makes of the arithmetic,
    // so the entry offset below is a scalar soffset and not a per-lane value
    // that would put every code load in a readfirstlane loop.
    const uint32_t nSE = SE1 - SE0;
    const uint32_t E0 = __builtin_amdgcn_readfirstlane(SE0 + ((kw * nSE) >> p.kw_shift));
    const uint32_t E1 = __builtin_amdgcn_readfirstlane(SE0 + (((kw + 1) * nSE) >> p.kw_shift));

    uint32_t *ldsM = reinterpret_cast<uint32_t *>(lds);  // [tr*16][Gp] s|b<<16, or [tr*16][Gp][2] f32
    unsigned char *img = lds + p.meta_bytes;              // [nT] tile images
    float *red = reinterpret_cast<float *>(lds + p.meta_bytes + p.img_bytes);
    float *sq = red + p.tr * KW * B * 16u;  // MLP: [wave][B] sums of x^2 over the split's columns

    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t *>(up_tile ? p.w2 : p.w), 0, int(p.w_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.s), 0, int(p.m_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t br =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.b), 0, int(p.m_bytes), kRsrcWord3);
    // The MLP form's up-matrix metadata. The 16-byte unit loads read one
    // matrix per unit; the per-value path (rows whose runs are not 16-byte
    // multiples) loads from both, the other matrix's through kOut (zeros),
    // and ORs them: there the row's matrix differs between lanes, and a
    // per-lane buffer resource would put every load in a readfirstlane loop.
    const __amdgpu_buffer_rsrc_t sr2 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(MLP ? p.s2 : p.s), 0, int(p.m_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t br2 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(MLP ? p.b2 : p.b), 0, int(p.m_bytes), kRsrcWord3);
    const uint32_t mat_rows = H * 16u;  // staged rows per matrix
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(p.x), 0, int(uint32_t(B) * p.cols * 4u), kRsrcWord3);

    // ---- 1. The split's x, requested first: at the start every workgroup
    // queues its loads behind those of the workgroups dispatched before it on
    // its CU, and nothing can be multiplied before x is staged. Item it = ((Tl*B + t)*4 + g)*4 + m covers the 8
    // columns (ST0 + Tl)*128 + 32g + 8m of RHS t (mfma_common.hpp). ----
    // Tiles whose images the first phase stages; with PH = 2 the rest follow
    // in the second phase into the same LDS, whose capacity is the larger.
    const uint32_t nT1 = PH == 2 ? min(p.phase_tiles, nT) : nT;
    const uint32_t nTimg = PH == 2 ? max(nT1, nT - nT1) : nT;
    const uint32_t items = nT1 * B * 16u;
    float xv[XI][8];
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const uint32_t it = uint32_t(tid) + uint32_t(i * nthr);
        load_x8(xv[i], xr, uint32_t(item_pos<B>(it).t), ST0 * kTileK + item_col<B>(it), p.cols, it < items);
    }
    // MLP: the norm weights of the same columns.
    [[maybe_unused]] float nv[MLP ? XI : 1][8];
    if constexpr (MLP) {
        const __amdgpu_buffer_rsrc_t nr =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p.norm), 0, int(p.cols * 4u), kRsrcWord3);
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const uint32_t it = uint32_t(tid) + uint32_t(i * nthr);
            load_x8(nv[i], nr, 0u, ST0 * kTileK + item_col<B>(it), p.cols, it < items);
        }
    }

    // ---- 2. Metadata of the band's rows over the split's groups: one run
    // per row and plane, as 16-byte loads when the rows are 16-byte aligned
    // (every checkpoint shape). A run covers groups [Ga, Gb): G0 rounded down
    // and G1 rounded up to whole 16-byte units, both inside the row (nG is a
    // multiple of VEC); the `lead` groups before G0 and those past G1 are
    // read and dropped, so splits may start at any entry. Rows past the
    // matrix read zeros through the buffer range check. ----
    // Thread tid loads column tid % 2^unit_shift of rows tid >> unit_shift,
    // + rstep, ... (2^unit_shift >= units per row: no division, and
    // consecutive lanes read consecutive 16 bytes of a row).
    const bool vec_meta = (nG * MB) % 16 == 0;
    const uint32_t lead = G0 % uint32_t(VEC);
    const uint32_t Ga = G0 - lead;
    const uint32_t Gb = (G1 + uint32_t(VEC) - 1) / uint32_t(VEC) * uint32_t(VEC);
    const uint32_t upr = vec_meta ? (Gb - Ga) / uint32_t(VEC) : 0u;  // units per row
    const uint32_t band_rows = p.tr * 16u;
    const uint32_t ucol = uint32_t(tid) & ((1u << p.unit_shift) - 1u);
    const uint32_t urow = uint32_t(tid) >> p.unit_shift;
    const uint32_t rstep = uint32_t(nthr) >> p.unit_shift;
    const bool ucol_ok = ucol < upr;
    // Staged row rl is matrix row band_row0 + rl (the MLP form: rows past
    // mat_rows are the up matrix's rows rl - mat_rows).
    auto mrow = [&](uint32_t rl) -> uint32_t { return band_row0 + (MLP && rl >= mat_rows ? rl - mat_rows : rl); };
    auto unit_off = [&](uint32_t rl) -> uint32_t { return (mrow(rl) * nG + Ga) * MB + ucol * 16u; };
    // One 16-byte unit of each plane; `up` (uniform) selects the MLP form's
    // up matrix.
    auto load_units = [&](bool up, uint32_t off, u4 &sv, u4 &bv) {
        sv = __builtin_amdgcn_raw_buffer_load_b128(up ? sr2 : sr, int(off), 0, 0);
        bv = __builtin_amdgcn_raw_buffer_load_b128(up ? br2 : br, int(off), 0, 0);
    };
    // Unrolled unit u's staged row: urow + u*rstep; in the MLP form the first
    // half of the units take gate rows urow + u*rstep and the second half the
    // up matrix's same rows (staged mat_rows further), so that every load
    // reads one matrix through a uniform resource.
    constexpr int kHalfUnits = kMetaUnits / 2;
    auto unit_row = [&](int u) -> uint32_t {
        if constexpr (MLP)
            return (u < kHalfUnits ? 0u : mat_rows) + urow + uint32_t(u % kHalfUnits) * rstep;
        else
            return urow + uint32_t(u) * rstep;
    };
    auto unit_live = [&](int u) -> bool {
        if constexpr (MLP)
            return urow + uint32_t(u % kHalfUnits) * rstep < mat_rows;
        else
            return urow + uint32_t(u) * rstep < band_rows;
    };
    u4 ms[kMetaUnits], mbv[kMetaUnits];
#pragma unroll
    for (int u = 0; u < kMetaUnits; ++u) {
        const uint32_t off = (ucol_ok && unit_live(u)) ? unit_off(unit_row(u)) : kOut;
        load_units(MLP && u >= kHalfUnits, off, ms[u], mbv[u]);
    }

    // ---- 3. The first P entries of codes. An entry is 128 contiguous bytes
    // of each of the tile's 16 rows, read with two 16-byte loads per lane:
    // rows 0-7 then 8-15, eight lanes per row; lanes r and r^8 swap one
    // piece through DPP after the loads land. ----
    const bool lo_half = r < 8;
    const uint32_t kp = BITS == 4 ? uint32_t(lg) : 2u * lg;          // 16-byte piece kept
    const uint32_t sp = BITS == 4 ? uint32_t(lg) + 4 : 2u * lg + 1;  // piece sent to lane r^8
    const uint32_t piece1 = lo_half ? kp : sp;
    const uint32_t piece2 = lo_half ? sp : kp;
    const uint32_t row_bytes = p.cols / 32 * (BITS * 4);
    const uint32_t rowA = tile_row0 + (r & 7), rowB = tile_row0 + 8 + (r & 7);
    // A lane's two pieces at entry 0 are per-lane offsets, kOut for rows past
    // the matrix; entry E adds E*128 as the wave-uniform soffset. Lanes sent
    // to kOut read zeros whatever the entry (kOut + E*128 stays below 2^32),
    // and in-range lanes stay inside their own row: E < E1 <= n_entries, and
    // in a row's partial last entry the pieces past the row's end go to kOut.
    // Entries past the wave's range (the ring's tail) read zeros.
    const uint32_t tail_bytes = row_bytes & 127u;  // bytes of a partial last entry (0: none)
    const uint32_t vA = rowA < p.rows ? rowA * row_bytes + 16 * piece1 : kOut;
    const uint32_t vB = rowB < p.rows ? rowB * row_bytes + 16 * piece2 : kOut;
    const uint32_t vAt = 16 * piece1 < tail_bytes ? vA : kOut;
    const uint32_t vBt = 16 * piece2 < tail_bytes ? vB : kOut;
    auto issue = [&](u4 (&c)[2], uint32_t E) {
        const bool live = E < E1;
        const bool last = tail_bytes != 0 && E + 1 == p.n_entries;
        const int so = int(E * 128u);
        c[0] = __builtin_amdgcn_raw_buffer_load_b128(wr, int(live ? (last ? vAt : vA) : kOut), so, kAuxStream);
        c[1] = __builtin_amdgcn_raw_buffer_load_b128(wr, int(live ? (last ? vBt : vB) : kOut), so, kAuxStream);
    };
    u4 ring[P][2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < P; ++j) {
        issue(ring[j], E0 + j);
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- 4. x as MFMA operand images (hi/lo f16, group sums, epilogue
    // factors), tile by tile, as soon as x has landed: x was requested
    // first and comes from L2, while the metadata behind it comes from HBM.
    // ----
    u4 *imgA = reinterpret_cast<u4 *>(img);
    float4 *imgS = reinterpret_cast<float4 *>(img + nTimg * TIMG_A);
    // MLP: each x[t]'s sum of squares over the split's columns, from the
    // staged items (items past the split read zeros), for 1/rms at the end.
    [[maybe_unused]] float xsq[MLP ? B : 1] = {};
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const uint32_t it = uint32_t(tid) + uint32_t(i * nthr);
        if (i > 0 && uint32_t(tid) - uint32_t(lane) + uint32_t(i * nthr) >= items) break;  // whole waves in or out
        if constexpr (MLP) {
            float q = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) q += xv[i][j] * xv[i][j];
            const uint32_t it_t = item_pos<B>(it).t;
#pragma unroll
            for (int t = 0; t < B; ++t) xsq[t] += it_t == uint32_t(t) ? q : 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) xv[i][j] *= nv[i][j];
        }
        stage_x_item<BITS, GROUP, B>(xv[i], it, it < items, lane, imgA, imgS);
    }
    // Each wave's sums of squares to LDS (with two phases, once the second
    // phase's items are added).
    auto put_sq = [&]() {
#pragma unroll
        for (int t = 0; t < (MLP ? B : 1); ++t) {
            float v = xsq[t];
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
            if (lane == 0) sq[wave * B + t] = v;
        }
    };
    if constexpr (MLP && PH == 1) put_sq();
    // ---- 5. Metadata to LDS. ----
    if (vec_meta) {
        // This thread's units hold groups g .. g+VEC-1 of their rows (g
        // relative to G0: negative in the lead); only groups in [0, G1 - G0)
        // are kept, which checks only a row's first and last unit.
        const uint32_t ng = G1 - G0;
        const int g = int(ucol * uint32_t(VEC)) - int(lead);
        const bool inner = ucol > 0 && ucol + 1 < upr;
        auto put = [&](uint32_t rl, const u4 &sv, const u4 &bv) {
            auto keep = [&](int gg) { return inner || (gg >= 0 && uint32_t(gg) < ng); };
            if constexpr (META == 0) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (keep(g + e)) {
                        uint32_t *dst = ldsM + (rl * Gp + uint32_t(g + e)) * 2;
                        dst[0] = sv[e];
                        dst[1] = bv[e];
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (keep(g + 2 * e)) ldsM[rl * Gp + uint32_t(g + 2 * e)] = __builtin_amdgcn_perm(bv[e], sv[e], 0x05040100u);
                    if (keep(g + 2 * e + 1))
                        ldsM[rl * Gp + uint32_t(g + 2 * e + 1)] = __builtin_amdgcn_perm(bv[e], sv[e], 0x07060302u);
                }
            }
        };
        if (ucol_ok) {
#pragma unroll
            for (int u = 0; u < kMetaUnits; ++u)
                if (unit_live(u)) put(unit_row(u), ms[u], mbv[u]);
            // Bands with more rows than the unrolled loads cover read the rest here.
            if constexpr (MLP) {
                for (uint32_t rl = urow + uint32_t(kHalfUnits) * rstep; rl < mat_rows; rl += rstep) {
                    u4 sv, bv;
                    load_units(false, unit_off(rl), sv, bv);
                    put(rl, sv, bv);
                    load_units(true, unit_off(rl + mat_rows), sv, bv);
                    put(rl + mat_rows, sv, bv);
                }
            } else {
                for (uint32_t rl = urow + uint32_t(kMetaUnits) * rstep; rl < band_rows; rl += rstep) {
                    u4 sv, bv;
                    load_units(false, unit_off(rl), sv, bv);
                    put(rl, sv, bv);
                }
            }
        }
    } else {
        const uint32_t ng = G1 - G0;
        for (uint32_t f = uint32_t(tid); f < p.tr * 16u * ng; f += uint32_t(nthr)) {
            const uint32_t rl = f / ng;
            const uint32_t g = f - rl * ng;
            const uint32_t off = (mrow(rl) * nG + G0 + g) * MB;
            const bool up_row = MLP && rl >= mat_rows;
            const uint32_t og = up_row ? kOut : off, ou = up_row ? off : kOut;
            if constexpr (META == 0) {
                uint32_t sv = __builtin_amdgcn_raw_buffer_load_b32(sr, int(og), 0, 0);
                uint32_t bv = __builtin_amdgcn_raw_buffer_load_b32(br, int(og), 0, 0);
                if constexpr (MLP) {
                    sv |= __builtin_amdgcn_raw_buffer_load_b32(sr2, int(ou), 0, 0);
                    bv |= __builtin_amdgcn_raw_buffer_load_b32(br2, int(ou), 0, 0);
                }
                ldsM[(rl * Gp + g) * 2] = sv;
                ldsM[(rl * Gp + g) * 2 + 1] = bv;
            } else {
                uint32_t sv = __builtin_amdgcn_raw_buffer_load_b16(sr, int(og), 0, 0);
                uint32_t bv = __builtin_amdgcn_raw_buffer_load_b16(br, int(og), 0, 0);
                if constexpr (MLP) {
                    sv |= __builtin_amdgcn_raw_buffer_load_b16(sr2, int(ou), 0, 0);
                    bv |= __builtin_amdgcn_raw_buffer_load_b16(br2, int(ou), 0, 0);
                }
                ldsM[rl * Gp + g] = (sv & 0xFFFFu) | (bv << 16);
            }
        }
    }
    // Groups of a partial last K tile past the matrix: zero entries (their
    // products are zero, and finite metadata keeps them so).
    {
        const uint32_t extra = nT * NGM - (G1 - G0);
        for (uint32_t f = uint32_t(tid); f < p.tr * 16u * extra; f += uint32_t(nthr)) {
            const uint32_t rl = f / extra;
            const uint32_t g = (G1 - G0) + (f - rl * extra);
            if constexpr (META == 0) {
                ldsM[(rl * Gp + g) * 2] = 0u;
                ldsM[(rl * Gp + g) * 2 + 1] = 0u;
            } else {
                ldsM[rl * Gp + g] = 0u;
            }
        }
    }

    // Zero sums and factors of absent RHS.
    stage_x_pads<GROUP, B>(nT1, tid, nthr, imgS);
    lds_barrier();

    // ---- 6. Stream the wave's entries. ----
    const LaneMap<GROUP, B> L(lane);
    const int t0 = L.t0;
    const uint32_t m_row = (ti * 16u + uint32_t(r)) * Gp + uint32_t(L.gD);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    h8 a[4] = {h8{}, h8{}, h8{}, h8{}};
    // The images of the current phase start at tile img_base (0, or nT1 in
    // the second phase of PH = 2); the metadata covers the whole split.
    uint32_t img_base = 0;
    auto compute = [&](const u4 (&c)[NLD], uint32_t Tl) {
        float sv, bv;
        meta_entry<META>(ldsM + (m_row + Tl * NGM) * (META == 0 ? 2 : 1), sv, bv);
        const uint32_t Ti = Tl - img_base;
        const float4 sx = imgS[(Ti * NGM + L.gD) * (HALF / 2) + t0 / 2];
        tile_product<BITS, META, GROUP, B>(c, L, imgA + Ti * 4 * (8 * B), sv, bv, sx, a, acc);
    };
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
    const uint32_t nE = E1 - E0;
    // One pass of the ring: the P entries from `base`, each multiplied once
    // landed and its slot refilled with the entry P further on. Every pass
    // issues the same loads, so the wait before each entry's product counts
    // only the loads behind it.
    auto pass = [&](uint32_t base) {
#pragma unroll
        for (int j = 0; j < P; ++j) {
            const uint32_t i = base + j;
            if (i < nE) {
                const uint32_t E = E0 + i;
                u4 kept, got;
                exchange(ring[j], kept, got);
                const uint32_t Tl = E * TPE - ST0;
                if constexpr (BITS == 4) {
                    const u4 c0[1] = {kept};
                    compute(c0, Tl);
                    if (E * 2 + 1 < p.tiles) {
                        const u4 c1[1] = {got};
                        compute(c1, Tl + 1);
                    }
                } else {
                    const u4 c[2] = {kept, got};
                    compute(c, Tl);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            issue(ring[j], E0 + i + P);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if constexpr (PH == 2) {
        // Two phases (every wave streams the same entries, so all meet the
        // barriers together). phase_entry is a multiple of P inside the
        // stream: the first phase ends with a whole pass, before which x of
        // tiles [nT1, nT) is requested, so it lands behind the ring's loads
        // without waiting for them. Once every wave has multiplied its last
        // first-phase entry, those x images replace the first phase's.
        const uint32_t pe = p.phase_entry;
        uint32_t base = 0;
        for (; base + P < pe; base += P) pass(base);
        const uint32_t items2 = (nT - nT1) * B * 16u;
        const uint32_t col2 = (ST0 + nT1) * kTileK;
        float x2[XI][8];
        [[maybe_unused]] float nv2[MLP ? XI : 1][8];
#pragma unroll
        for (int i2 = 0; i2 < XI; ++i2) {
            const uint32_t it = uint32_t(tid) + uint32_t(i2 * nthr);
            load_x8(x2[i2], xr, uint32_t(item_pos<B>(it).t), col2 + item_col<B>(it), p.cols, it < items2);
        }
        if constexpr (MLP) {
            const __amdgpu_buffer_rsrc_t nr =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p.norm), 0, int(p.cols * 4u), kRsrcWord3);
#pragma unroll
            for (int i2 = 0; i2 < XI; ++i2) {
                const uint32_t it = uint32_t(tid) + uint32_t(i2 * nthr);
                load_x8(nv2[i2], nr, 0u, col2 + item_col<B>(it), p.cols, it < items2);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        pass(base);
        lds_barrier();
#pragma unroll
        for (int i2 = 0; i2 < XI; ++i2) {
            const uint32_t it = uint32_t(tid) + uint32_t(i2 * nthr);
            if (i2 > 0 && uint32_t(tid) - uint32_t(lane) + uint32_t(i2 * nthr) >= items2) break;
            if constexpr (MLP) {
                float q = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) q += x2[i2][j] * x2[i2][j];
                const uint32_t it_t = item_pos<B>(it).t;
#pragma unroll
                for (int t = 0; t < B; ++t) xsq[t] += it_t == uint32_t(t) ? q : 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) x2[i2][j] *= nv2[i2][j];
            }
            stage_x_item<BITS, GROUP, B>(x2[i2], it, it < items2, lane, imgA, imgS);
        }
        if constexpr (MLP) put_sq();
        stage_x_pads<GROUP, B>(nT - nT1, tid, nthr, imgS);
        lds_barrier();
        img_base = nT1;
        for (base = pe; base < nE; base += P) pass(base);
    } else {
        for (uint32_t base = 0; base < nE; base += P) pass(base);
    }

    // ---- 7. Combine hi/lo slots and quant groups, add the KW partial sums
    // of each row in wave order, then finish the band across splits. ----
    float v0, v1;
    combine_slots<GROUP>(acc, v0, v1);
    constexpr int WRITERS = 4 / NGM;  // lane groups holding distinct RHS pairs
    if (lg < WRITERS) {
        float *dst = red + (size_t(wave) * B) * 16u + uint32_t(r);
        if (t0 < B) dst[size_t(t0) * 16u] = v0;
        if (t0 + 1 < B) dst[size_t(t0 + 1) * 16u] = v1;
    }
    __syncthreads();
    // One thread per output row and RHS (the MLP form: per gate row, whose
    // up row is H tiles further down the band).
    const uint32_t outs = H * 16u * B;
    const uint32_t tt = uint32_t(tid) / (16u * B);  // tile within the band (of the gate rows)
    const uint32_t t = (uint32_t(tid) / 16u) % B;
    const uint32_t rr = uint32_t(tid) % 16u;
    const uint32_t row = band_row0 + tt * 16u + rr;
    const bool live = uint32_t(tid) < outs && row < p.rows;
    // Elected finishers (plans over several rounds of workgroups): every
    // split publishes, and the band's last workgroup to arrive (an arrival
    // counter elects it) finishes, so no workgroup waits for one that is not
    // resident. Otherwise the band's last split finishes and the others only
    // publish. Threads without an output row leave here unless the election
    // needs them at its barriers.
    const bool elect = p.elect != 0 && p.ns > 1;
    if (!live && !elect) return;
    auto wave_sum_of = [&](uint32_t tile) -> float {
        const float *src = red + (size_t(tile * KW) * B + t) * 16u + rr;
        float sum = src[0];
        for (uint32_t k = 1; k < KW; ++k) sum += src[size_t(k) * B * 16u];
        return sum;
    };
    const float v = live ? wave_sum_of(tt) : 0.f;
    const size_t oy = size_t(t) * p.rows + row;
    const size_t stride = size_t(B) * p.rows;
    // Slot sets: one per publishing split (all ns when elected, else ns-1).
    const uint32_t nsets = elect ? p.ns : p.ns - 1;
    // Reads slot set k's value for oy once its epoch is this launch's;
    // past the host's spin limit it gives up: the caller writes NaN and
    // reports the band in the status word, which the host turns into a
    // failed command at its finish.
    // The finisher requests the slots it needs kFetchChunk splits at a time
    // (one round trip per chunk where the other splits have all published:
    // `fetch`), then polls only the words that lack the launch's epoch
    // (`settle`).
    auto fetch = [&](unsigned long long *q) -> unsigned long long {
        return __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto settle = [&](unsigned long long word, unsigned long long *q, bool &ok) -> float {
        for (uint32_t spin = 0; uint32_t(word >> 32) != p.wait_epoch; ++spin) {
            if (spin >= p.spin_limit) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            word = fetch(q);
        }
        return __uint_as_float(uint32_t(word));
    };
    auto slot = [&](uint32_t k) { return p.partial + size_t(k) * stride + oy; };
    auto report = [&](bool ok) {
        if (!ok && p.status) __hip_atomic_store(p.status, 0x80000000u | band, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    };
    auto publish_at = [&](unsigned long long *q, float value) {
        const unsigned long long word = (static_cast<unsigned long long>(p.epoch) << 32) | __float_as_uint(value);
        __hip_atomic_store(q, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto publish = [&](uint32_t k, float value) { publish_at(slot(k), value); };
    // The election, after this workgroup's slots are published (every
    // thread calls it): whether this workgroup finishes the band. The counter
    // only elects; a finisher takes each slot once it carries the launch's
    // epoch, so no ordering between the slot stores and the increments is
    // needed. The finisher returns the counter to zero (every other split of
    // the band has incremented it by then).
    auto elected = [&]() -> bool {
        __syncthreads();  // every wave is past its reads of red and sq
        int *flag = reinterpret_cast<int *>(red);
        if (tid == 0) {
            const uint32_t prev = __hip_atomic_fetch_add(&p.counters[band], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = prev + 1 == p.ns;
            if (last) __hip_atomic_store(&p.counters[band], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *flag = last ? 1 : 0;
        }
        __syncthreads();
        return *flag != 0;
    };
    if constexpr (MLP) {
        // Slot sets [2*k] (gate) and [2*k + 1] (up) of publishing split k,
        // then their sums of squares [k][band][B]; the finisher adds each in
        // split order, its own sums in its split's place.
        const float vu = live ? wave_sum_of(tt + H) : 0.f;
        float ss = 0.f;
        for (uint32_t wv = 0; wv < p.tr * KW; ++wv) ss += sq[wv * B + t];
        // Split k's sum of squares for this band and RHS (ns > 1 only).
        auto sq_slot = [&](uint32_t k) {
            return p.partial + size_t(2) * nsets * stride + (size_t(k) * p.nbands + band) * B + t;
        };
        auto publish_all = [&]() {
            publish(2 * split, v);
            publish(2 * split + 1, vu);
            if (tt == 0 && rr == 0) publish_at(sq_slot(split), ss);
        };
        if (elect) {
            if (live) publish_all();
            if (!elected() || !live) return;
        } else if (!finisher) {
            publish_all();
            return;
        }
        bool ok = true;
        float g = v, u = vu;
        if (p.ns > 1) {
            float sg = 0.f, su = 0.f, sx = 0.f;
            for (uint32_t k0 = 0; k0 < p.ns; k0 += kFetchChunk) {
                unsigned long long wg[kFetchChunk], wu[kFetchChunk], wx[kFetchChunk];
#pragma unroll
                for (uint32_t j = 0; j < kFetchChunk; ++j) {
                    const uint32_t k = k0 + j;
                    const bool other = k < p.ns && k != split;
                    wg[j] = other ? fetch(slot(2 * k)) : 0ull;
                    wu[j] = other ? fetch(slot(2 * k + 1)) : 0ull;
                    wx[j] = other ? fetch(sq_slot(k)) : 0ull;
                }
#pragma unroll
                for (uint32_t j = 0; j < kFetchChunk; ++j) {
                    const uint32_t k = k0 + j;
                    if (k >= p.ns) break;
                    const float kg = k == split ? v : settle(wg[j], slot(2 * k), ok);
                    const float ku = k == split ? vu : settle(wu[j], slot(2 * k + 1), ok);
                    const float kx = k == split ? ss : settle(wx[j], sq_slot(k), ok);
                    sg = k == 0 ? kg : sg + kg;
                    su = k == 0 ? ku : su + ku;
                    sx = k == 0 ? kx : sx + kx;
                }
            }
            g = sg;
            u = su;
            ss = sx;
        }
        const float inv = 1.0f / sqrtf(ss / float(p.cols) + p.eps);
        const float gn = g * inv;
        p.y[oy] = ok ? gn * (1.0f / (1.0f + expf(-gn))) * (u * inv) : __builtin_nanf("");
        report(ok);
        return;
    } else {
        float y = v;
        // The residual form's r, requested before the cross-split sum so that
        // its round trip overlaps the slot reads (with elected finishers
        // every split requests it; the one elected uses it). In place (y is
        // r) each element is read and then written by the same thread.
        [[maybe_unused]] float rv = 0.f;
        if constexpr (FUSE == 1)
            if (live && (elect || split + 1 == p.ns)) rv = p.r[oy];
        if (p.ns > 1) {
            if (elect) {
                if (live) publish(split, v);
                if (!elected() || !live) return;
            } else if (split + 1 < p.ns) {
                publish(split, v);
                return;
            }
            // The finisher: every split's sum in split order, its own in its
            // place. Each slot is this thread's alone, so with reset_slots it
            // is cleared once taken (the finisher's own too when it was
            // published), leaving the workspace zero for the next launch
            // (which may then reuse the same epoch).
            bool ok = true;
            float sum = 0.f;
            for (uint32_t k0 = 0; k0 < p.ns; k0 += kFetchChunk) {
                unsigned long long w[kFetchChunk];
#pragma unroll
                for (uint32_t j = 0; j < kFetchChunk; ++j)
                    w[j] = k0 + j < p.ns && k0 + j != split ? fetch(slot(k0 + j)) : 0ull;
#pragma unroll
                for (uint32_t j = 0; j < kFetchChunk; ++j) {
                    const uint32_t k = k0 + j;
                    if (k >= p.ns) break;
                    const float kv = k == split ? v : settle(w[j], slot(k), ok);
                    sum = k == 0 ? kv : sum + kv;
                }
            }
            if (p.reset_slots)
                for (uint32_t k = 0; k < nsets; ++k)
                    __hip_atomic_store(slot(k), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            y = ok ? sum : __builtin_nanf("");
            report(ok);
        }
        p.y[oy] = FUSE == 1 ? rv + y : y;
    }
}

template <int BITS, int META, int GROUP, int B, int XI, int P, int FUSE, int PH>
hipError_t launch_inst(const BandParams &p, const TilePlan &pl, hipStream_t stream) {
    auto kernel = affine_band_kernel<BITS, META, GROUP, B, XI, P, FUSE, PH>;
    if (pl.lds > 65536) {
        const hipError_t e = raise_lds_limit(reinterpret_cast<const void *>(kernel), pl.lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, dim3(pl.nbands * pl.ns), dim3(pl.tr * pl.kw * 64), pl.lds, stream, p);
    return hipGetLastError();
}

template <int BITS, int META, int GROUP, int B, int XI>
hipError_t launch_xi(const BandParams &p, const TilePlan &pl, hipStream_t stream) {
    const int fuse = p.w2 != nullptr ? 2 : p.r != nullptr ? 1 : 0;
    if (pl.phases == 2) {
        // Every wave must stream the same entries to meet the phase barriers.
        if (pl.ns != 1 || pl.kw != 1) return hipErrorInvalidValue;
        if (pl.ring >= 3) {
            if (fuse == 2) return launch_inst<BITS, META, GROUP, B, XI, 3, 2, 2>(p, pl, stream);
            return fuse == 1 ? launch_inst<BITS, META, GROUP, B, XI, 3, 1, 2>(p, pl, stream)
                             : launch_inst<BITS, META, GROUP, B, XI, 3, 0, 2>(p, pl, stream);
        }
        if (fuse == 2) return launch_inst<BITS, META, GROUP, B, XI, 2, 2, 2>(p, pl, stream);
        return fuse == 1 ? launch_inst<BITS, META, GROUP, B, XI, 2, 1, 2>(p, pl, stream)
                         : launch_inst<BITS, META, GROUP, B, XI, 2, 0, 2>(p, pl, stream);
    }
    if (pl.ring >= 3) {
        if (fuse == 2) return launch_inst<BITS, META, GROUP, B, XI, 3, 2, 1>(p, pl, stream);
        return fuse == 1 ? launch_inst<BITS, META, GROUP, B, XI, 3, 1, 1>(p, pl, stream)
                         : launch_inst<BITS, META, GROUP, B, XI, 3, 0, 1>(p, pl, stream);
    }
    if (fuse == 2) return launch_inst<BITS, META, GROUP, B, XI, 2, 2, 1>(p, pl, stream);
    return fuse == 1 ? launch_inst<BITS, META, GROUP, B, XI, 2, 1, 1>(p, pl, stream)
                     : launch_inst<BITS, META, GROUP, B, XI, 2, 0, 1>(p, pl, stream);
}

// x items per thread: the smallest compiled count that covers the plan's.
// Every unrolled item issues its loads (dead ones read zeros), so the
// metric shapes get exact counts: 2 at B=1 and 5 at B=3 (5120x17408, three
// splits), each 0.15-0.2 us faster than rounding up to 4 and 8; 3 serves
// 17408x5120 at B=1 (two splits), plain and MLP form.
constexpr uint32_t xi_instance(uint32_t xi) { return xi <= 2 ? 2 : xi <= 3 ? 3 : xi <= 4 ? 4 : xi <= 5 ? 5 : 8; }

template <int BITS, int META, int GROUP, int B>
hipError_t launch_b(const BandParams &p, const TilePlan &pl, hipStream_t stream) {
    switch (xi_instance(pl.xi)) {
        case 2: return launch_xi<BITS, META, GROUP, B, 2>(p, pl, stream);
        case 3: return launch_xi<BITS, META, GROUP, B, 3>(p, pl, stream);
        case 4: return launch_xi<BITS, META, GROUP, B, 4>(p, pl, stream);
        case 5: return launch_xi<BITS, META, GROUP, B, 5>(p, pl, stream);
        default: return launch_xi<BITS, META, GROUP, B, 8>(p, pl, stream);
    }
}

template <int BITS, int META, int GROUP>
hipError_t launch_group(const BandParams &p, const TilePlan &pl, uint32_t batch, hipStream_t stream) {
    constexpr int MAXB = (16 / (kTileK / GROUP)) / 2;
    switch (batch) {
        case 1: return launch_b<BITS, META, GROUP, 1>(p, pl, stream);
        case 2: return launch_b<BITS, META, GROUP, 2>(p, pl, stream);
        case 3:
            if constexpr (MAXB >= 3) return launch_b<BITS, META, GROUP, 3>(p, pl, stream);
            break;
        case 4:
            if constexpr (MAXB >= 4) return launch_b<BITS, META, GROUP, 4>(p, pl, stream);
            break;
        default: break;
    }
    return hipErrorInvalidValue;
}

template <int BITS, int META, int GROUP>
const void *instance_group(uint32_t batch, uint32_t xi, uint32_t ring, bool mlp, uint32_t phases) {
    constexpr int MAXB = (16 / (kTileK / GROUP)) / 2;
    auto pick = [&](auto bconst) -> const void * {
        constexpr int B = decltype(bconst)::value;
        auto by_ring = [&](auto xconst) -> const void * {
            constexpr int XI = decltype(xconst)::value;
            if (phases == 2 && mlp)
                return ring >= 3 ? reinterpret_cast<const void *>(affine_band_kernel<BITS, META, GROUP, B, XI, 3, 2, 2>)
                                 : reinterpret_cast<const void *>(affine_band_kernel<BITS, META, GROUP, B, XI, 2, 2, 2>);
            if (phases == 2)
                return ring >= 3 ? reinterpret_cast<const void *>(affine_band_kernel<BITS, META, GROUP, B, XI, 3, 0, 2>)
                                 : reinterpret_cast<const void *>(affine_band_kernel<BITS, META, GROUP, B, XI, 2, 0, 2>);
            if (mlp)
                return ring >= 3 ? reinterpret_cast<const void *>(affine_band_kernel<BITS, META, GROUP, B, XI, 3, 2, 1>)
                                 : reinterpret_cast<const void *>(affine_band_kernel<BITS, META, GROUP, B, XI, 2, 2, 1>);
            return ring >= 3 ? reinterpret_cast<const void *>(affine_band_kernel<BITS, META, GROUP, B, XI, 3, 0, 1>)
                             : reinterpret_cast<const void *>(affine_band_kernel<BITS, META, GROUP, B, XI, 2, 0, 1>);
        };
        switch (xi_instance(xi)) {
            case 2: return by_ring(std::integral_constant<int, 2>{});
            case 3: return by_ring(std::integral_constant<int, 3>{});
            case 4: return by_ring(std::integral_constant<int, 4>{});
            case 5: return by_ring(std::integral_constant<int, 5>{});
            default: return by_ring(std::integral_constant<int, 8>{});
        }
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

}  // namespace

namespace band {

template <int BITS, int META>
hipError_t launch_meta(const BandParams &p, const TilePlan &pl, uint32_t group, uint32_t batch,
                       hipStream_t stream) {
    switch (group) {
        case 32: return launch_group<BITS, META, 32>(p, pl, batch, stream);
        case 64: return launch_group<BITS, META, 64>(p, pl, batch, stream);
        case 128: return launch_group<BITS, META, 128>(p, pl, batch, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int BITS, int META>
const void *instance_meta(uint32_t group, uint32_t batch, uint32_t xi, uint32_t ring, bool mlp, uint32_t phases) {
    switch (group) {
        case 32: return instance_group<BITS, META, 32>(batch, xi, ring, mlp, phases);
        case 64: return instance_group<BITS, META, 64>(batch, xi, ring, mlp, phases);
        case 128: return instance_group<BITS, META, 128>(batch, xi, ring, mlp, phases);
        default: return nullptr;
    }
}

template hipError_t launch_meta<QMR_BAND_BITS, QMR_BAND_META>(const BandParams &, const TilePlan &, uint32_t, uint32_t,
                                                               hipStream_t);
template const void *instance_meta<QMR_BAND_BITS, QMR_BAND_META>(uint32_t, uint32_t, uint32_t, uint32_t, bool,
                                                                   uint32_t);

}  // namespace band

#else  // the planner and the launch entry
namespace {

using namespace mfma;
using band::BandParams;
using band::instance_meta;
using band::kMaxThreads;
using band::launch_meta;

// First entry of split s (the last split ends at n_entries): splits differ
// by at most one entry.
uint32_t host_split_begin(uint32_t s, uint32_t ns, uint32_t n_entries) {
    if (s >= ns) return n_entries;
    return uint32_t((uint64_t(s) * n_entries) / ns);
}

// log2 of the smallest power of two >= the 16-byte metadata units of any
// split's row run (the kernel's Ga..Gb), as the kernel computes them.
uint32_t meta_unit_shift(const AffineArgs &a, uint32_t ns, uint32_t n_entries) {
    const uint32_t tpe = 8 / a.bits, ngm = kTileK / a.group;
    const uint32_t tiles = (a.cols + kTileK - 1) / kTileK, ng = a.cols / a.group;
    const uint32_t vec = a.meta == Meta::F32 ? 4 : 8;
    uint32_t most = 1;
    for (uint32_t sp = 0; sp < ns; ++sp) {
        const uint32_t g0 = host_split_begin(sp, ns, n_entries) * tpe * ngm;
        const uint32_t g1 = std::min(std::min(host_split_begin(sp + 1, ns, n_entries) * tpe, tiles) * ngm, ng);
        const uint32_t ga = g0 - g0 % vec, gb = (g1 + vec - 1) / vec * vec;
        most = std::max(most, (gb - ga) / vec);
    }
    uint32_t shift = 0;
    while ((1u << shift) < most) ++shift;
    return shift;
}

uint32_t log2_exact(uint32_t v) {
    uint32_t k = 0;
    while ((1u << k) < v) ++k;
    return k;
}

const void *instance(const AffineArgs &a, uint32_t xi, uint32_t ring, uint32_t phases = 1) {
    const int meta = static_cast<int>(a.meta);
    const bool mlp = a.up_w != nullptr;
    if (a.bits == 4) {
        if (meta == 0) return instance_meta<4, 0>(a.group, a.batch, xi, ring, mlp, phases);
        if (meta == 1) return instance_meta<4, 1>(a.group, a.batch, xi, ring, mlp, phases);
        return instance_meta<4, 2>(a.group, a.batch, xi, ring, mlp, phases);
    }
    if (meta == 0) return instance_meta<8, 0>(a.group, a.batch, xi, ring, mlp, phases);
    if (meta == 1) return instance_meta<8, 1>(a.group, a.batch, xi, ring, mlp, phases);
    return instance_meta<8, 2>(a.group, a.batch, xi, ring, mlp, phases);
}

// Resident workgroups per CU for an instance, block size and dynamic LDS,
// as the runtime computes them from registers and LDS; cached.
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

bool affine_tile_supported(const AffineArgs &a) {
    if (a.up_w && (a.residual || a.norm == nullptr || !a.up_s || !a.up_b)) return false;
    if (a.up_w && (reinterpret_cast<uintptr_t>(a.up_w) & 15) != 0) return false;
    if (a.bits != 4 && a.bits != 8) return false;
    if (a.group != 32 && a.group != 64 && a.group != 128) return false;
    const uint32_t maxb = (16 / (kTileK / a.group)) / 2;
    if (a.batch < 1 || a.batch > maxb) return false;
    if (a.cols == 0 || a.rows == 0 || a.cols % 32 != 0 || a.cols % a.group != 0) return false;
    if ((reinterpret_cast<uintptr_t>(a.w) & 15) != 0) return false;
    const uint64_t w_bytes = uint64_t(a.rows) * a.cols * a.bits / 8;
    const uint64_t m_bytes = uint64_t(a.rows) * (a.cols / a.group) * (a.meta == Meta::F32 ? 4 : 2);
    return w_bytes < (1ull << 31) && m_bytes < (1ull << 31) && uint64_t(a.batch) * a.cols * 4 < (1ull << 31);
}

TilePlan plan_affine_tile(const AffineArgs &a, const DeviceLimits &lim, uint32_t force_kw, uint32_t force_tr,
                          uint32_t force_ns, uint32_t force_ring, uint32_t force_phases) {
    TilePlan pl;
    if (!affine_tile_supported(a)) return pl;
    const uint32_t row_tiles = (a.rows + 15) / 16;
    const uint32_t row_bytes = a.cols / 32 * (a.bits * 4);
    const uint32_t n_entries = (row_bytes + 127) / 128;
    const uint32_t ngm = kTileK / a.group;
    const uint32_t tpe = 8 / a.bits;
    const uint32_t tiles = (a.cols + kTileK - 1) / kTileK;
    const uint32_t mb = a.meta == Meta::F32 ? 4 : 2;
    const uint32_t cus = lim.num_cus > 0 ? uint32_t(lim.num_cus) : 256u;
    const bool mlp = a.up_w != nullptr;
    const size_t timg = size_t(4) * 4 * 2 * a.batch * 16 + size_t(ngm) * ((16 / ngm / 2) / 2) * 16;
    const double wbytes = double(a.rows) * row_bytes + 2.0 * a.rows * (a.cols / a.group) * mb;
    // Candidates: ring depth, K splits, tiles per band, waves per tile. Every
    // workgroup must be resident in one round (a second round repeats the
    // start-up latency). Score, fitted to timings on MI355X of every feasible
    // plan of six shapes (5120x17408, 17408x5120 and 12288x4096 Q4,
    // 17408x5120 Q8, 5120x5120 Q4 and Q8) at B=1..4:
    //   0.25 |log2(waves / two per SIMD)|
    //   + log2(workgroups per CU rounded up / the even share)
    //   + 2 x bytes read from L2 (once per band) / weight bytes: every band
    //     converts its x, which the stream waits for
    //   + 0.25 |log2(codes in flight per CU / 36 KB)|, with waves per CU x
    //     ring x 2 KB entries in flight: the stream slows with less (latency
    //     not covered) and with more (at 5120x17408 B=1: 12.2 us with 30 KB,
    //     11.9 with 45, 12.3 with 60)
    //   + 0.1 for a two-entry ring
    //   + 4 splits / entries per row: short splits read their rows'
    //     metadata in short runs.
    // Against the best measured plan of each of the 24 cases, two sweeps on
    // two runs: the previous weights (0.5, 1, 1, 1, 0.1, 0) lost 9.9 and
    // 10.4 us in total, these 3.9 and 3.8 (17408x5120 Q4 at B=2..4 takes
    // three splits of 8-tile bands: 15.9-17.0 -> 15.0-15.4 us; 12288x4096
    // at B=1 and B=2 single-split 4-tile bands of two waves: 9.1 -> 8.9,
    // 10.0 -> 9.1 us).
    // Where no plan fits one round (a 151936-row vocabulary head), a second
    // pass takes single-split bands, whose workgroups never wait on each
    // other, so any number of rounds is safe: the tallest band, one wave per
    // tile, and the ring whose codes in flight per CU (resident waves x ring
    // x 2 KB) come closest to 48 KB. The MLP form takes this pass through
    // the rule after it, or when forced. Measured at 151936x5120 Q4/g64,
    // two boxes: B=1 76.7-80.4 us (tr 8, kw 1, ring 2; two workgroups per
    // CU) against 86.4-89.8 for the row-owning kernel and 80.9-81.9 with
    // ring 3; B=3 95.0-96.7 (ring 3; one 106 KB workgroup per CU) against
    // 95.1-97.0 and 98.8-99.2 with ring 2, before x was staged in two phases
    // there (below). Two or three splits over several rounds measured slower
    // at both batches.
    double best = 1e30;
    for (int pass = 0; pass < 2 && pl.kw == 0; ++pass) {
        // Several rounds: single-split bands; split bands with elected
        // finishers (no workgroup waits) and the MLP form only when forced.
        if (pass == 1 && mlp && !force_ns) break;
        for (uint32_t ring : {2u, 3u}) {
            if (force_ring && ring != force_ring) continue;
            for (uint32_t ns = 1; ns <= (force_ns ? band::kBandSplits : band::kPlannedSplits); ++ns) {
                if (force_ns && ns != force_ns) continue;
                if (pass == 1 && ns != 1 && !force_ns) continue;
                if (ns > n_entries) continue;
                uint32_t max_se = 0;
                bool empty = false;
                for (uint32_t sp = 0; sp < ns; ++sp) {
                    const uint32_t e0 = host_split_begin(sp, ns, n_entries);
                    const uint32_t e1 = host_split_begin(sp + 1, ns, n_entries);
                    if (e1 <= e0) empty = true;
                    else max_se = std::max(max_se, e1 - e0);
                }
                if (empty) continue;
                const uint32_t max_tiles = std::min(max_se * tpe, tiles);
                for (uint32_t tr : {1u, 2u, 4u, 8u}) {
                    if (force_tr && tr != force_tr) continue;
                    // The MLP form: tr/2 gate tiles and tr/2 up tiles per band.
                    if (mlp && tr < 2) continue;
                    const uint32_t h = mlp ? tr / 2 : tr;  // row tiles per matrix in a band
                    if (h > 1 && (h / 2) * 16 >= a.rows) continue;
                    const uint32_t nbands = (row_tiles + h - 1) / h;
                    for (uint32_t kw : {1u, 2u, 4u, 8u}) {
                        if (force_kw && kw != force_kw) continue;
                        const uint32_t threads = tr * kw * 64;
                        if (threads > uint32_t(kMaxThreads) || kw > max_se) continue;
                        if ((1u << meta_unit_shift(a, ns, n_entries)) > threads) continue;
                        const uint32_t items = max_tiles * a.batch * 16;
                        const uint32_t xi = (items + threads - 1) / threads;
                        if (xi > 8) continue;
                        const uint32_t gp = (max_tiles * ngm) | 1u;
                        const size_t meta = (size_t(tr) * 16 * gp * 4 * (a.meta == Meta::F32 ? 2 : 1) + 15) & ~size_t(15);
                        const size_t img = size_t(max_tiles) * timg;
                        // The MLP form: the finishers' sums of squares after the
                        // reduction area.
                        const size_t lds = meta + img + size_t(tr * kw) * a.batch * 16 * 4 +
                                           (mlp ? size_t(tr * kw) * a.batch * 4 : 0);
                        if (lds > lim.max_lds_per_block) continue;
                        const double wgs = double(nbands) * ns;
                        const uint32_t resident = resident_per_cu(instance(a, xi, ring), threads, lds);
                        double score;
                        if (pass == 0) {
                            if (wgs > double(resident) * cus) continue;
                            const double waves = wgs * tr * kw;
                            const double per_cu = std::ceil(wgs / cus) / (wgs / cus);
                            score = 0.25 * std::fabs(std::log2(waves / (2.0 * 4 * cus)));
                            score += std::log2(per_cu);
                            score += 2.0 * double(nbands) * a.batch * a.cols * 4.0 / (wbytes * (mlp ? 2 : 1));
                            score += 0.25 * std::fabs(std::log2(waves / cus * ring * 2048.0 / 36864.0));
                            score += ring == 2 ? 0.1 : 0.0;
                            score += 4.0 * ns / n_entries;
                        } else {
                            const double flight = double(resident) * tr * kw * ring * 2048.0;
                            score = double(8 / tr) + double(kw) + std::fabs(std::log2(flight / 49152.0));
                        }
                        if (score < best - 1e-9) {
                            best = score;
                            pl.kw = kw;
                            pl.tr = tr;
                            pl.ns = ns;
                            pl.nbands = nbands;
                            pl.n_entries = n_entries;
                            pl.tiles = tiles;
                            pl.gp = gp;
                            pl.meta_bytes = uint32_t(meta);
                            pl.img_bytes = uint32_t(img);
                            pl.xi = xi;
                            pl.ring = ring;
                            pl.lds = lds;
                            pl.elect = pass == 1 && ns > 1;
                        }
                    }
                }
            }
        }
    }
    // The MLP form where no plan fits one round (B >= 2 at the 27B gate/up
    // shape 2 x 17408x5120): single-split bands of two gate and two up
    // tiles with a two-entry ring, whose workgroups never wait on each
    // other, so any number of rounds is safe (x in two phases where that
    // raises the resident workgroups, below); where that has no plan (B=4
    // there: more x items per thread than compiled), 8-tile bands in two
    // splits with elected finishers. Measured on MI355X, six shuffled
    // rounds of 200 launches, medians: B=2 28.9 us against 30.2 for the
    // split-K kernel, B=3 30.5 against 31.3, B=4 31.8 against 32.0 (8-tile
    // single-split bands: 31.2, 32.6 and 41.3 us; a three-entry ring at
    // B=3: 37.3).
    if (pl.kw == 0 && mlp && !force_kw && !force_tr && !force_ns && !force_ring) {
        pl = plan_affine_tile(a, lim, 1, 4, 1, 2, force_phases);
        if (pl.kw == 0) pl = plan_affine_tile(a, lim, 1, 8, 2, 2, force_phases);
        return pl;
    }
    // Short streams: fewer than 8 entries per wave run faster with half the
    // row tiles per band (more, shorter workgroups) where x costs little to
    // convert against the codes: at one RHS, and for 8-bit codes (twice the
    // bytes per staged column). Measured on one box, every feasible plan
    // timed: 5120x5120 Q8 9.18 -> 8.36 us, Q4 7.74 -> 7.54 us at B=1; at B=3
    // Q8 9.37 -> 9.23 and, on another box, 9.62 -> 9.25 us, while halving
    // cost Q4 0.57 us. The longer streams of the other fitted shapes (8-20
    // entries per wave) keep their plans.
    if (pl.kw > 0 && !mlp && (a.batch == 1 || a.bits == 8) && pl.tr >= 4 && !force_kw && !force_tr && !force_ns &&
        !force_ring && pl.n_entries < 8 * pl.ns * pl.kw) {
        const TilePlan half = plan_affine_tile(a, lim, pl.kw, pl.tr / 2, pl.ns, pl.ring, force_phases);
        if (half.kw > 0) pl = half;
    }
    // Streams of at most four entries per wave take the two-entry ring: a
    // deeper ring requests nearly the whole stream up front. Measured on
    // MI355X, every feasible plan timed twice in shuffled order: 5120x5120
    // Q4/g64 (3.3 entries per wave) 7.52 -> 7.18 us at B=1 and 8.20 -> 7.80
    // at B=3; Q8 of the same shape (6.7 entries per wave) and the metric
    // shape (11.3) keep the three-entry ring, their fastest.
    if (pl.kw > 0 && !mlp && pl.ring == 3 && !force_ring && pl.n_entries <= 4 * pl.ns * pl.kw) {
        const TilePlan two = plan_affine_tile(a, lim, pl.kw, pl.tr, pl.ns, 2, force_phases);
        if (two.kw > 0) pl = two;
    }
    // Two-phase x staging for single-split plans of one wave per tile that
    // take several rounds of workgroups (matrices too tall for one round):
    // half the x images in LDS lets more workgroups share a CU, so one
    // workgroup's x conversion overlaps another's stream. Taken when it
    // raises the resident workgroups per CU: at 151936x5120 Q4/g64 (8-tile
    // bands, 1187 workgroups) B=2 and B=3 go from one workgroup per CU to
    // two, measured on MI355X at 92 -> 83 us (B=2) and 95.5 -> 88.8 us (B=3),
    // three alternating runs each. Where residency stays the same the
    // phase switch only costs (B=1 there: 71.7 -> 75.9 us forced), and at
    // B=4 the halved images still leave one workgroup per CU.
    if (pl.kw == 1 && pl.ns == 1 && force_phases != 1 && pl.n_entries >= 4) {
        const uint32_t threads = pl.tr * 64;
        struct Phased {
            bool ok = false;
            uint32_t pe = 0, xi = 0, resident = 0;
            size_t img = 0, lds = 0;
        };
        auto phased = [&](uint32_t ring) {
            Phased f;
            // The second phase starts at a whole pass of the ring.
            f.pe = std::max(ring, pl.n_entries / 2 / ring * ring);
            if (f.pe >= pl.n_entries) return f;
            const uint32_t nt1 = std::min(f.pe * tpe, tiles);
            const uint32_t cap = std::max(nt1, tiles - nt1);
            f.xi = (cap * a.batch * 16 + threads - 1) / threads;
            f.img = size_t(cap) * timg;
            f.lds = size_t(pl.meta_bytes) + f.img + size_t(pl.tr) * a.batch * 16 * 4 +
                    (mlp ? size_t(pl.tr) * a.batch * 4 : 0);
            if (f.xi > 8 || f.lds > lim.max_lds_per_block) return f;
            f.resident = resident_per_cu(instance(a, f.xi, ring, 2), threads, f.lds);
            f.ok = f.resident > 0;
            return f;
        };
        Phased f = phased(pl.ring);
        if (f.ok) {
            const uint32_t r1 = resident_per_cu(instance(a, pl.xi, pl.ring), threads, pl.lds);
            const bool rounds = double(pl.nbands) > double(r1) * cus;
            if (force_phases == 2 || (rounds && f.resident > r1)) {
                // The ring is picked again for the phased residency, by the
                // same rule as the several-round pass (codes in flight per
                // CU closest to 48 KB). Measured on the 151936x5120 head at
                // B=3, five shuffled rounds of 40 launches, min / median:
                // 80.7 / 83.5 us with the two-entry ring against 82.8 / 85.8
                // with three (B=2 level: 77.9 / 80.2 against 78.6 / 79.7).
                if (!force_ring) {
                    auto off = [&](uint32_t ring, const Phased &g) {
                        return std::fabs(std::log2(double(g.resident) * pl.tr * ring * 2048.0 / 49152.0));
                    };
                    const uint32_t other = pl.ring == 3 ? 2 : 3;
                    const Phased g = phased(other);
                    if (g.ok && off(other, g) < off(pl.ring, f) - 1e-9) {
                        pl.ring = other;
                        f = g;
                    }
                }
                pl.phases = 2;
                pl.phase_entry = f.pe;
                pl.xi = f.xi;
                pl.img_bytes = uint32_t(f.img);
                pl.lds = f.lds;
            }
        }
    }
    return pl;
}

size_t affine_tile_workspace(const TilePlan &pl, const AffineArgs &a) {
    if (pl.ns <= 1) return 0;
    const size_t sets = pl.elect ? pl.ns : pl.ns - 1;  // publishing splits
    if (a.up_w)  // gate and up sums per row, then each band's sums of x^2
        return sets * (size_t(2) * a.rows + pl.nbands) * a.batch * sizeof(unsigned long long);
    return sets * a.batch * a.rows * sizeof(unsigned long long);
}

hipError_t launch_affine_tile(const AffineArgs &a, const TilePlan &pl, unsigned long long *partial, uint32_t *counters,
                              uint32_t epoch, const TileWait &wait, hipStream_t stream) {
    if (pl.kw == 0) return hipErrorInvalidValue;
    if (pl.ns > 1 && partial == nullptr) return hipErrorInvalidValue;
    if (pl.elect && pl.ns > 1 && counters == nullptr) return hipErrorInvalidValue;
    BandParams p;
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
    p.partial = partial;
    p.epoch = epoch;
    // A forced give-up waits for a tag no split of this launch publishes,
    // with a short bound, so that every workgroup still exits.
    p.wait_epoch = wait.force_give_up ? epoch + 0x40000000u : epoch;
    p.spin_limit = wait.force_give_up ? 64u : 1u << 22;
    p.status = wait.status;
    p.reset_slots = wait.reset_slots && a.up_w == nullptr ? 1u : 0u;
    p.elect = pl.elect && pl.ns > 1 ? 1u : 0u;
    p.counters = counters;
    p.rows = a.rows;
    p.cols = a.cols;
    p.w_bytes = uint32_t(uint64_t(a.rows) * a.cols * a.bits / 8);
    p.m_bytes = uint32_t(uint64_t(a.rows) * (a.cols / a.group) * (a.meta == Meta::F32 ? 4 : 2));
    p.tr = pl.tr;
    p.kw = pl.kw;
    p.ns = pl.ns;
    p.nbands = pl.nbands;
    p.n_entries = pl.n_entries;
    p.tiles = pl.tiles;
    p.gp = pl.gp;
    p.meta_bytes = pl.meta_bytes;
    p.img_bytes = pl.img_bytes;
    for (uint32_t k = 0; k <= band::kBandSplits; ++k) p.split_e[k] = host_split_begin(k, pl.ns, pl.n_entries);
    p.kw_shift = log2_exact(pl.kw);
    p.unit_shift = meta_unit_shift(a, pl.ns, pl.n_entries);
    p.phase_entry = pl.phases == 2 ? pl.phase_entry : pl.n_entries;
    p.phase_tiles = std::min(p.phase_entry * (8u / a.bits), pl.tiles);
    if (pl.phases == 2 && (pl.phase_entry == 0 || pl.phase_entry >= pl.n_entries || pl.phase_entry % pl.ring != 0))
        return hipErrorInvalidValue;
    const int meta = static_cast<int>(a.meta);
    if (a.bits == 4) {
        if (meta == 0) return launch_meta<4, 0>(p, pl, a.group, a.batch, stream);
        if (meta == 1) return launch_meta<4, 1>(p, pl, a.group, a.batch, stream);
        return launch_meta<4, 2>(p, pl, a.group, a.batch, stream);
    }
    if (meta == 0) return launch_meta<8, 0>(p, pl, a.group, a.batch, stream);
    if (meta == 1) return launch_meta<8, 1>(p, pl, a.group, a.batch, stream);
    return launch_meta<8, 2>(p, pl, a.group, a.batch, stream);
}

#endif

}  // namespace qmr

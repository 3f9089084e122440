// Launch interface between the host runtime (runtime.cpp) and the HIP
// kernels (affine_rows.hip, affine_mfma.hip, affine_gemv.hip, affine_tile.hip,
// dense_mfma.hip, misc_kernels.hip, wide_mfma.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "contract.hpp"

namespace qmr {

// One packed-affine product: y[t][r] = sum_c (q*s + b) * x[t][c] for
// t < batch (token-major x [batch][cols], y [batch][rows]).
struct AffineArgs {
    const uint32_t *w;  // [rows][cols*bits/32] packed codes, little-endian fields
    const void *s;      // [rows][cols/group] metadata (F32 or 16-bit patterns)
    const void *b;
    const float *x;
    float *y;
    uint32_t rows, cols, bits, group, batch;
    Meta meta;
    // Fused forms (null when unused).
    //  - residual: y = residual + W x, added in the final store (may alias y).
    //  - MLP (up_w set): w/s/b are the gate matrix and up_w/up_s/up_b the up
    //    matrix of the same shape and format; x[t] is RMS-normalised with the
    //    `norm` weights and `eps`, and y[t] = silu(gate x) * (up x).
    const float *residual = nullptr;
    const uint32_t *up_w = nullptr;
    const void *up_s = nullptr;
    const void *up_b = nullptr;
    const float *norm = nullptr;
    float eps = 0.f;
};

// Tiling of the GEMV/block kernel. A workgroup has 8 half-wave row slots;
// `ks` slots share a row group and split its K rounds, each slot owns `rr`
// rows. rr/ks = 0 lets the planner choose.
struct GemvPlan {
    int rr = 0;
    int ks = 0;
};

// Raises a kernel's dynamic-LDS limit on the current device to `bytes`
// (launches above 64 KB need it): once per kernel, device and larger size,
// under a lock, so that device handles used from different threads do not
// race on it.
hipError_t raise_lds_limit(const void *kernel, size_t bytes);

struct DeviceLimits {
    size_t max_lds_per_block;  // bytes of LDS one workgroup may allocate
    int num_cus;
};

// VALU GEMV / small-block kernel (batch 1..4, group 32/64/128, Q4/Q8).
hipError_t launch_affine_gemv(const AffineArgs &a, GemvPlan plan, const DeviceLimits &lim,
                              hipStream_t stream);
// Reference-arithmetic kernel for any group size (also reference mode).
hipError_t launch_affine_generic(const AffineArgs &a, hipStream_t stream);
// Row dequantisation y[c] = q*s + b (bit-exact RN32).
hipError_t launch_embed_affine(const uint32_t *w, const void *s, const void *b, Meta meta,
                               uint32_t row, uint32_t cols, uint32_t bits, uint32_t group,
                               float *y, hipStream_t stream);
// Dense F16 weights: matvec / block and embedding row.
hipError_t launch_dense_f16(const uint16_t *w, const float *x, float *y, uint32_t rows,
                            uint32_t cols, uint32_t batch, hipStream_t stream);
hipError_t launch_embed_f16(const uint16_t *w, uint32_t row, uint32_t cols, float *y,
                            hipStream_t stream);
// y[i] = x[i] for i < n (x == y allowed only as the identical view).
hipError_t launch_copy_f32(const float *x, float *y, uint32_t n, int num_cus, hipStream_t stream);
// p[i] = 0 for i < n (a fill kernel: safe to capture into a graph).
hipError_t launch_zero_u32(uint32_t *p, uint32_t n, hipStream_t stream);
// One wave that returns after `ticks` of the device's real-time counter.
hipError_t launch_delay(unsigned long long ticks, hipStream_t stream);
// Geometry of read_checksum: workgroups of 256 threads (0 = about 48 KB per
// workgroup), 16-byte loads per thread in flight (1, 2, 4 or 8; 0 = 4),
// non-temporal loads (1), plain (0) or the default (-1: non-temporal).
struct ReadPlan {
    uint32_t workgroups = 0;
    uint32_t unroll = 0;
    int nt = -1;
};
// One streaming read of three views (byte sizes, multiples of 4); out holds
// kChecksumSlots u32 whose XOR is the XOR of every word read.
hipError_t launch_read_checksum(const void *a, uint32_t na, const void *b, uint32_t nb, const void *c, uint32_t nc,
                                uint32_t *out, const ReadPlan &plan, hipStream_t stream);
// A last arriver's wait on the other K splits' {value, epoch} slots (the
// row-band, split-K and dense kernels).
struct TileWait {
    // Device-visible word that a last arriver which gives up sets to
    // 0x80000000 | band (row-band kernel: its band's workgroups were not all
    // resident), 0xC0000000 | band (split-K kernel) or 0xA0000000 | band
    // (dense kernel); null: no report (the outputs are NaN either way).
    uint32_t *status = nullptr;
    // The last arriver clears each slot it took (row-band: plain and residual
    // forms; split-K and dense: every form), so that a workspace that was
    // zero stays zero and the next launch may reuse the same epoch.
    bool reset_slots = false;
    // Testing: the last arriver waits for a tag no split publishes and gives
    // up after a short bound; every workgroup still exits.
    bool force_give_up = false;
};

// Streaming GEMV / small block on the matrix cores (batch 1..4; Q4/Q8;
// group 32/64/128 with 2*batch <= 16*group/128). See affine_mfma.hip.
struct MfmaPlan {
    uint32_t rt = 0;      // waves (16-row tiles) per workgroup; 0 = unsupported
    uint32_t nbands = 0;  // row bands
    uint32_t ns = 0;      // K splits across workgroups
    uint32_t tiles = 0;   // 128-column K tiles
    uint32_t tps = 0;     // K tiles per split
    bool pairs = false;   // 16-bit metadata staged with 32-bit loads
    size_t lds = 0;       // dynamic LDS bytes per workgroup
    uint32_t rounds = 0;  // rounds of resident workgroups the grid takes
};
bool affine_mfma_supported(const AffineArgs &a);
// force_ns > 0 (tuning hook) keeps only that number of K splits.
MfmaPlan plan_affine_mfma(const AffineArgs &a, const DeviceLimits &lim, uint32_t force_ns = 0);
// Workspace bytes the plan needs for cross-workgroup partial sums (0 if none).
size_t affine_mfma_workspace(const MfmaPlan &pl, const AffineArgs &a);
// `slots` holds affine_mfma_workspace bytes (64-bit slots: a partial counts
// only when its epoch matches); `epoch` must differ from the previous
// launch's that used the same slots, unless those slots were cleared;
// `counters` holds pl.nbands zeroed u32 (the kernel returns them to zero).
hipError_t launch_affine_mfma(const AffineArgs &a, const MfmaPlan &pl, unsigned long long *slots,
                              uint32_t *counters, uint32_t epoch, const TileWait &wait, hipStream_t stream);

// Dense F16 matvec / block (batch 1..4) on the matrix cores: row bands of
// 16-row tiles, K in ns splits whose epoch-tagged sums an elected finisher
// adds. See dense_mfma.hip.
struct DensePlan {
    uint32_t rt = 0;      // 16-row tiles per workgroup; 0 = unsupported
    uint32_t kw = 0;      // waves per tile (contiguous K runs of the split)
    uint32_t ring = 0;    // 128-byte entries in flight per wave (4 or 8)
    uint32_t nbands = 0;  // row bands
    uint32_t ns = 0;      // K splits across workgroups
    uint32_t tiles = 0;   // 128-column K tiles
    uint32_t tps = 0;     // K tiles per split
    uint32_t xi = 0;      // x items staged per thread
    size_t lds = 0;       // dynamic LDS bytes per workgroup
    double cost_us = 0;   // the planner's time estimate
};
// Fields the tuning hook pins (0 = the planner's choice).
struct DenseForce {
    uint32_t ring = 0, kw = 0, rt = 0, ns = 0;
};
// 16-byte aligned weights, cols % 32 == 0, 1..4 RHS, views below 2 GiB.
bool dense_mfma_supported(const uint16_t *w, uint32_t rows, uint32_t cols, uint32_t batch);
// Pinned fields that no feasible plan has fall back to the planner's plan.
// The planner scores every feasible plan with a cost model fitted to MI355X
// timings and keeps the cheapest.
DensePlan plan_dense_mfma(uint32_t rows, uint32_t cols, uint32_t batch, const DeviceLimits &lim,
                          const DenseForce &force = DenseForce{});
size_t dense_mfma_workspace(const DensePlan &pl, uint32_t rows, uint32_t batch);
// Estimated time (us) of the vector-ALU dense kernels on the same product,
// for the choice between the two.
double dense_valu_cost(uint32_t rows, uint32_t cols, uint32_t batch);
// `slots` (dense_mfma_workspace bytes) and `counters` (pl.nbands zeroed u32)
// as for launch_affine_mfma; both may be null when pl.ns == 1.
hipError_t launch_dense_mfma(const uint16_t *w, const float *x, float *y, uint32_t rows, uint32_t cols,
                             uint32_t batch, const DensePlan &pl, unsigned long long *slots, uint32_t *counters,
                             uint32_t epoch, const TileWait &wait, hipStream_t stream);

// Streaming GEMV / small block on the matrix cores with every workgroup
// owning whole rows (no cross-workgroup reduction). See affine_rows.hip.
struct RowsPlan {
    uint32_t rt = 0;         // 16-row tiles per workgroup; 0 = unsupported
    uint32_t kw = 0;         // K waves per tile
    uint32_t j = 0;          // entries per wave per staged chunk
    uint32_t nbands = 0;     // workgroups
    uint32_t n_entries = 0;  // 128-byte entries per row
    uint32_t n_chunks = 0;   // ceil(n_entries / (kw * j))
    bool pairs = false;      // 16-bit metadata staged with 32-bit loads
    size_t stage_bytes = 0;  // one LDS staging buffer
    size_t lds = 0;          // dynamic LDS bytes per workgroup
};
bool affine_rows_supported(const AffineArgs &a);
// force_rt/force_kw (both nonzero) pin the workgroup shape and force_j the
// chunk depth; zeros leave the choice to the planner.
// The MLP form's tiling: gate and up tiles of the same rows in one workgroup
// (even rt, the first rt/2 tiles from the gate matrix).
RowsPlan plan_affine_mlp(const AffineArgs &a, const DeviceLimits &lim, uint32_t force_rt = 0,
                         uint32_t force_kw = 0, uint32_t force_j = 0);
RowsPlan plan_affine_rows(const AffineArgs &a, const DeviceLimits &lim, uint32_t force_rt = 0,
                          uint32_t force_kw = 0, uint32_t force_j = 0);
hipError_t launch_affine_rows(const AffineArgs &a, const RowsPlan &pl, hipStream_t stream);

// Streaming GEMV / small block on the matrix cores over row bands of 16-row
// tiles: each band's K range in ns long splits across workgroups and KW
// contiguous per-wave runs inside one; the band's last split adds the
// others' epoch-tagged partial sums. See affine_tile.hip.
struct TilePlan {
    uint32_t kw = 0;          // waves per row tile; 0 = unsupported
    uint32_t tr = 0;          // row tiles per band (workgroup)
    uint32_t ns = 0;          // K splits across workgroups
    uint32_t nbands = 0;      // row bands
    uint32_t n_entries = 0;   // 128-byte entries per row
    uint32_t tiles = 0;       // 128-column K tiles
    uint32_t gp = 0;          // LDS pitch of a row's metadata
    uint32_t meta_bytes = 0;  // LDS bytes of the staged metadata
    uint32_t img_bytes = 0;   // LDS bytes of the staged x images
    uint32_t xi = 0;          // x items staged per thread
    uint32_t ring = 0;        // code entries in flight per wave (2 or 3)
    size_t lds = 0;           // dynamic LDS bytes per workgroup
    bool elect = false;       // every split publishes; an arrival counter elects each band's finisher
    uint32_t phases = 1;      // 2: x images staged in two halves (single split, one wave per tile)
    uint32_t phase_entry = 0; // with phases == 2: the first entry of the second half
};
bool affine_tile_supported(const AffineArgs &a);
// Zeros leave the choice to the planner; force_phases 1 keeps one phase of
// x staging, 2 takes two where the plan allows it.
TilePlan plan_affine_tile(const AffineArgs &a, const DeviceLimits &lim, uint32_t force_kw = 0,
                          uint32_t force_tr = 0, uint32_t force_ns = 0, uint32_t force_ring = 0,
                          uint32_t force_phases = 0);
// Workspace bytes for the partial-sum slots (0 when ns == 1).
size_t affine_tile_workspace(const TilePlan &pl, const AffineArgs &a);
// `partial` holds affine_tile_workspace bytes (64-bit slots: a slot counts
// only when its epoch matches); `epoch` must differ from the previous
// launch's that used the same slots, unless those slots were cleared.
// `counters` holds pl.nbands zeroed u32 when pl.elect (the kernel returns
// them to zero); otherwise it may be null.
hipError_t launch_affine_tile(const AffineArgs &a, const TilePlan &pl, unsigned long long *partial,
                              uint32_t *counters, uint32_t epoch, const TileWait &wait, hipStream_t stream);

// Wide block on MFMA (Q4/g64, F32 or BF16 metadata, batch up to 256): a prep
// launch converts x into per-group images in `workspace` (wide_mfma_workspace
// bytes), then the contraction launch. See wide_mfma.hip.
bool wide_mfma_supported(const AffineArgs &a);
size_t wide_mfma_workspace(const AffineArgs &a);
hipError_t launch_wide_mfma(const AffineArgs &a, unsigned char *workspace, const DeviceLimits &lim,
                            hipStream_t stream);
// Host-side walk of every code, x-fragment and group-sum load the wide
// contraction kernel issues for a shape with nrt row tiles per block: the
// largest end (offset + size) of the in-range loads in the code view and in
// the image workspace, beside the two extents.
struct WideExtent {
    uint64_t code_end, code_extent, image_end, image_extent;
};
WideExtent wide_address_extent(uint32_t rows, uint32_t cols, uint32_t n, uint32_t nrt);

// The plan the GEMV launcher would use (for tests and tuning reports).
GemvPlan plan_affine_gemv(const AffineArgs &a, GemvPlan forced, const DeviceLimits &lim);

}  // namespace qmr

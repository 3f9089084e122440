// Wide block (chunked prefill) on the matrix cores: Q4/g64 weights times up
// to 256 RHS, y[t][r] = sum_c (q[r,c]*s[r,g] + b[r,g]) * x[t][c]. This is a
// real dense contraction (MFMA-bound), computed in the factored form
//     y[t][r] = sum_g ( s[r,g] * D[r,t,g] + b[r,g] * S[t,g] ),
//     D[r,t,g] = sum_{c in g} q[r,c] * x[t,c],  S[t,g] = sum_{c in g} x[t,c],
// with exact integer codes (f16 subnormals, as in mfma_common.hpp) and x
// split into hi/lo f16 parts, so D is accurate to about 2^-22 and the scale
// and bias are applied in FP32.
//
// Two launches:
//   1. wide_prep_kernel converts x once: for every (quant group g, block of
//      64 columns) it writes an "image" of exactly what the main kernel's LDS
//      needs: the hi/lo MFMA operands of the 64 columns for the two 32-column
//      K steps of the group (rows padded to 144 bytes so that operand reads
//      are free of bank conflicts), the column sums S and a power-of-two
//      scale 2^e taken from the block's max |x|.
//   2. wide_mfma_kernel: a workgroup (8 waves, 4 x 2) owns 128 rows x 64
//      columns. Per quant group it needs the 128 rows' codes (4 KB) and the
//      group's image (20 KB), staged in LDS (two buffers) from registers
//      that are loaded kLead groups ahead (three 16-byte units per thread
//      per group; the look-ahead covers the load latency); metadata (s, b)
//      arrives eight groups at a time. Each wave computes 32 rows x 32
//      columns: per group and K step, 2 code fragments (unpacked once, used
//      for 2 column tiles x hi/lo) and 4 activation fragments, 8 MFMAs; the
//      group's epilogue adds s*2^e*D + b*S into the FP32 accumulators.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.hpp"
#include "mfma_common.hpp"

namespace qmr {
namespace {

using namespace mfma;

constexpr int kPrepThreads = 256;
constexpr int kWideThreads = 256;  // 4 waves: 2 row halves x 2 column halves
constexpr int kColBlock = 64;         // columns per workgroup and per image
constexpr int kRowBlock = 128;        // rows per workgroup
constexpr int kImgColPitch = 144;     // bytes per column of one K step (hi 64, lo 64, pad 16)
constexpr int kImgStep = kColBlock * kImgColPitch;  // one K step of the image
constexpr int kImgS = 2 * kImgStep;                 // offset of S[64] (f32)
constexpr int kImgFac = kImgS + kColBlock * 4;      // offset of the scale factor (f32)
constexpr int kImgBytes = 20480;      // image size: five 4 KB copies per workgroup
constexpr int kCodeBytes = kRowBlock * 32;          // one group of codes: 128 rows x 32 B
constexpr int kStageBytes = kCodeBytes + kImgBytes;  // one LDS buffer (two in use)
constexpr int kLead = 3;              // groups held in registers ahead of LDS
constexpr int kRT = (kRowBlock / 16) / (kWideThreads / 128);  // 16-row tiles per wave
constexpr int kStageUnits = kStageBytes / (kWideThreads * 16);  // 16-byte units per thread per group
static_assert(kStageUnits * kWideThreads * 16 == kStageBytes, "stage copy shape");
static_assert(kCodeBytes == 4 * 64 * 16, "codes are the first four waves' first unit");
constexpr int kMetaGroups = 8;        // metadata arrives 8 groups per copy
static_assert(kImgFac + 4 <= kImgBytes, "image layout");

struct WideParams {
    const uint32_t *w;
    const void *s;
    const void *b;
    const float *x;
    float *y;
    const unsigned char *img;  // [G][NCB] images of kImgBytes
    uint32_t rows, cols, n;    // n = RHS count
    uint32_t ncb;              // column blocks
    uint32_t nrb;              // row blocks
    uint32_t w_bytes, m_bytes, img_bytes;  // extents of the views
};

// ---- 1. Activation images. grid (G, NCB), 256 threads: thread -> column
// tid/4 of the block, 16 K values (tid%4) of the group. ----
__global__ __launch_bounds__(kPrepThreads) void wide_prep_kernel(WideParams p) {
    __shared__ float red[kPrepThreads / 64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const uint32_t g = blockIdx.x, cb = blockIdx.y;
    const uint32_t c_local = uint32_t(tid) >> 2, sg = uint32_t(tid) & 3;
    const uint32_t t = cb * kColBlock + c_local;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(p.x), 0, int(p.n * p.cols * 4u), kRsrcWord3);
    float xv[2][8];
    const uint32_t k0 = g * 64 + sg * 16;
    load_x8(xv[0], xr, t, k0, p.cols, t < p.n);
    load_x8(xv[1], xr, t, k0 + 8, p.cols, t < p.n);
    float sum = 0.f, mx = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            sum += xv[h][j];
            mx = fmaxf(mx, fabsf(xv[h][j]));
        }
    group_reduce<4>(sum, mx);  // the column's 64 values (4 consecutive lanes)
    // Block max over the 64 columns.
    float m = mx;
#pragma unroll
    for (int o = 4; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const uint32_t mb = __float_as_uint(m);
    int e = 0;
    if (mb != 0u && mb < 0x7F800000u) {
        e = int(mb >> 23) - 127 - 14;  // max * 2^-e in [2^14, 2^15) for normal max
        e = e < -100 ? -100 : (e > 100 ? 100 : e);
    }
    const float sc = __uint_as_float(uint32_t(127 - e) << 23);
    unsigned char *img = const_cast<unsigned char *>(p.img) + (size_t(g) * p.ncb + cb) * kImgBytes;
    // This thread's 16 values are K step sg/2, chunks kq = 2*(sg%2) and +1.
    const uint32_t ks = sg >> 1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t kq = 2 * (sg & 1) + h;
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
            const float v0 = xv[h][k_of<4>(2 * e2)] * sc;
            const float v1 = xv[h][k_of<4>(2 * e2 + 1)] * sc;
            const h2 hh = __builtin_convertvector(f2{v0, v1}, h2);
            const h2 ll = __builtin_convertvector(f2{v0 - static_cast<float>(hh.x), v1 - static_cast<float>(hh.y)}, h2);
            hw[e2] = __builtin_bit_cast(uint32_t, hh);
            lw[e2] = __builtin_bit_cast(uint32_t, ll);
        }
        u4 *dst = reinterpret_cast<u4 *>(img + ks * kImgStep + c_local * kImgColPitch + kq * 16);
        dst[0] = u4{hw[0], hw[1], hw[2], hw[3]};
        dst[4] = u4{lw[0], lw[1], lw[2], lw[3]};  // +64 bytes: the lo part
    }
    if (sg == 0) reinterpret_cast<float *>(img + kImgS)[c_local] = sum;
    if (tid == 0) reinterpret_cast<float *>(img + kImgFac)[0] = __uint_as_float(uint32_t(127 + kCodeExp<4> + e) << 23);
}

__device__ __forceinline__ bool gi_last(uint32_t g) { return g % kMetaGroups == kMetaGroups - 1; }

// One Q4 word (8 codes) as the B operand of one MFMA, in k_of order.
__device__ __forceinline__ h8 unpack_word(uint32_t wd) {
    const u4 c[1] = {u4{wd, 0u, 0u, 0u}};
    return unpack<4>(c, 0);
}

// ---- 2. The contraction. grid (ceil(rows/128), NCB), 256 threads. ----
template <int META>
__global__ __launch_bounds__(kWideThreads) void wide_mfma_kernel(WideParams p) {
    constexpr int MB = META == 0 ? 4 : 2;                         // metadata bytes
    constexpr int META_BYTES = kRowBlock * kMetaGroups * MB;      // one array (s or b), one chunk
    constexpr int META_UNITS = 2 * META_BYTES / 16;               // 16-byte pieces, s then b
    constexpr int META_ITERS = (META_UNITS + kWideThreads - 1) / kWideThreads;
    constexpr int PER_ROW = kMetaGroups * MB / 16;                // 16-byte pieces per row
    constexpr int L = kLead;
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char *meta_lds = lds + 2 * kStageBytes;  // [2 chunks][s, b][128 rows][8 groups]
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const uint32_t wr = uint32_t(wave) >> 1, wc = uint32_t(wave) & 1;
    // XCD-aware tile order: workgroup i runs on XCD i % 8, so the column
    // blocks of one row block (which share its codes) and the row blocks
    // sharing a column block's images are placed on the same XCD and meet
    // in its L2.
    const uint32_t xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
    const uint32_t cb = slot % p.ncb;
    const uint32_t rb = (slot / p.ncb) * 8 + xcd;
    if (rb >= p.nrb) return;
    const uint32_t row0 = rb * kRowBlock;
    const uint32_t G = p.cols / 64;
    const uint32_t row_bytes = p.cols / 2;
    const uint32_t m_pitch = G * MB;  // metadata bytes per row
    const __amdgpu_buffer_rsrc_t wr_ =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(p.w), 0, int(p.w_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t ir =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char *>(p.img), 0, int(p.img_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.s), 0, int(p.m_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t br =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.b), 0, int(p.m_bytes), kRsrcWord3);

    // Staging registers: this thread's kStageUnits 16-byte units of group
    // g's LDS stage (unit q = tid + k*512 sits at byte 16q: units 0-255 are
    // the codes, 128 rows x 32 bytes, the rest the image), L groups ahead;
    // metadata one 8-group chunk ahead. Per-thread offsets are fixed; the
    // group moves only the uniform (scalar) offset. Rows past the matrix
    // read the last row (their results are never written).
    const bool code_thread = tid < kCodeBytes / 16;  // the first four waves
    const uint32_t code_off = min(row0 + (uint32_t(tid) >> 1), p.rows - 1) * row_bytes + (tid & 1) * 16;
    struct Staged {
        u4 u[kStageUnits];
    };
    auto load = [&](Staged &st, uint32_t g) {
        if (g >= G) return;
        const uint32_t img_base = (g * p.ncb + cb) * kImgBytes;
#pragma unroll
        for (int k = 0; k < kStageUnits; ++k) {
            const uint32_t q = uint32_t(tid) + k * kWideThreads;
            if (k == 0 && code_thread)
                st.u[k] = __builtin_amdgcn_raw_buffer_load_b128(wr_, int(code_off), int(g * 32), 0);
            else
                st.u[k] = __builtin_amdgcn_raw_buffer_load_b128(ir, int(q * 16 - kCodeBytes), int(img_base), 0);
        }
    };
    auto store = [&](const Staged &st, uint32_t g) {
        unsigned char *stage = lds + (g & 1) * kStageBytes;
#pragma unroll
        for (int k = 0; k < kStageUnits; ++k)
            *reinterpret_cast<u4 *>(stage + (uint32_t(tid) + k * kWideThreads) * 16) = st.u[k];
    };
    // Metadata piece q of [s rows][b rows] (each row = the chunk's 8 groups)
    // lands at 16q in the chunk's LDS buffer.
    u4 meta[META_ITERS];
    uint32_t meta_off[META_ITERS];
    bool meta_s[META_ITERS];
#pragma unroll
    for (int o = 0; o < META_ITERS; ++o) {
        const uint32_t q = uint32_t(tid) + o * kWideThreads;
        const uint32_t a = q / (META_BYTES / 16);
        const uint32_t idx = q - a * (META_BYTES / 16);
        meta_s[o] = a == 0;
        meta_off[o] = min(row0 + idx / PER_ROW, p.rows - 1) * m_pitch + (idx % PER_ROW) * 16;
    }
    auto load_meta = [&](uint32_t chunk) {
        if (chunk * kMetaGroups >= G) return;
#pragma unroll
        for (int o = 0; o < META_ITERS; ++o) {
            const uint32_t q = uint32_t(tid) + o * kWideThreads;
            if (q >= uint32_t(META_UNITS)) continue;
            const int soff = int(chunk * (kMetaGroups * MB));
            meta[o] = meta_s[o] ? __builtin_amdgcn_raw_buffer_load_b128(sr, int(meta_off[o]), soff, 0)
                                : __builtin_amdgcn_raw_buffer_load_b128(br, int(meta_off[o]), soff, 0);
        }
    };
    auto store_meta = [&](uint32_t chunk) {
        unsigned char *mb = meta_lds + (chunk & 1) * 2 * META_BYTES;
#pragma unroll
        for (int o = 0; o < META_ITERS; ++o) {
            const uint32_t q = uint32_t(tid) + o * kWideThreads;
            if (q < uint32_t(META_UNITS)) *reinterpret_cast<u4 *>(mb + q * 16) = meta[o];
        }
    };

    f4 acc[kRT][2], d[kRT][2];
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) acc[rt][ct] = d[rt][ct] = f4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](uint32_t g) {
        const unsigned char *stage = lds + (g & 1) * kStageBytes;
        const unsigned char *img = stage + kCodeBytes;
        const unsigned char *mb = meta_lds + ((g / kMetaGroups) & 1) * 2 * META_BYTES;
#pragma unroll
        for (uint32_t ks = 0; ks < 2; ++ks) {
            h8 bq[kRT], ax[2][2];
#pragma unroll
            for (int rt = 0; rt < kRT; ++rt) {
                const uint32_t rl = wr * (kRT * 16) + rt * 16 + r16;
                bq[rt] = unpack_word(*reinterpret_cast<const uint32_t *>(stage + rl * 32 + (ks * 4 + kq) * 4));
            }
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const unsigned char *col = img + ks * kImgStep + (wc * 32 + ct * 16 + r16) * kImgColPitch + kq * 16;
                ax[ct][0] = __builtin_bit_cast(h8, *reinterpret_cast<const u4 *>(col));
                ax[ct][1] = __builtin_bit_cast(h8, *reinterpret_cast<const u4 *>(col + 64));
            }
#pragma unroll
            for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    d[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[ct][0], bq[rt], d[rt][ct], 0, 0, 0);
                    d[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[ct][1], bq[rt], d[rt][ct], 0, 0, 0);
                }
        }
        // Epilogue: acc += s * 2^e * D + b * S (lane: row r16 of each row
        // tile, columns 4*kq .. 4*kq+3 of each column tile).
        const float fac = *reinterpret_cast<const float *>(img + kImgFac);
        float4 S[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
            S[ct] = *reinterpret_cast<const float4 *>(img + kImgS + (wc * 32 + ct * 16 + 4 * kq) * 4);
        const uint32_t gi = g % kMetaGroups;
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
            const uint32_t rl = wr * (kRT * 16) + rt * 16 + r16;
            float sv, bv;
            if constexpr (META == 0) {
                sv = reinterpret_cast<const float *>(mb)[rl * kMetaGroups + gi];
                bv = reinterpret_cast<const float *>(mb + META_BYTES)[rl * kMetaGroups + gi];
            } else {
                sv = meta_f32<META>(reinterpret_cast<const uint16_t *>(mb)[rl * kMetaGroups + gi]);
                bv = meta_f32<META>(reinterpret_cast<const uint16_t *>(mb + META_BYTES)[rl * kMetaGroups + gi]);
            }
            const float sf = sv * fac;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const float Sv[4] = {S[ct].x, S[ct].y, S[ct].z, S[ct].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc[rt][ct][e] = __builtin_fmaf(sf, d[rt][ct][e], acc[rt][ct][e]);
                    acc[rt][ct][e] = __builtin_fmaf(bv, Sv[e], acc[rt][ct][e]);
                }
                d[rt][ct] = f4{0.f, 0.f, 0.f, 0.f};
            }
        }
    };

    // Prologue: metadata chunk 0 and group 0 into LDS, groups 1..L loading.
    Staged st[L];
    load_meta(0);
    load(st[0], 0);
    store_meta(0);
    store(st[0], 0);
    load_meta(1);
#pragma unroll
    for (int j = 0; j < L; ++j) load(st[j], uint32_t(j) + 1);
    lds_barrier();

    // Group g: multiply from LDS buffer g%2, move group g+1 (register set
    // g%L) into the other buffer, refill that set with group g+1+L.
    // Metadata chunk c+1 moves into LDS while chunk c's last group is
    // multiplied; chunk c+2 then starts loading.
    for (uint32_t g0 = 0; g0 < G; g0 += L) {
#pragma unroll
        for (int j = 0; j < L; ++j) {
            const uint32_t g = g0 + j;
            if (g < G) {
                compute(g);
                if (g + 1 < G) {
                    store(st[j], g + 1);
                    load(st[j], g + 1 + L);
                }
                if (gi_last(g) && g + 1 < G) {
                    store_meta(g / kMetaGroups + 1);
                    load_meta(g / kMetaGroups + 2);
                }
                lds_barrier();
            }
        }
    }

    // y[t][r]: lane holds row r16 of each row tile and columns 4*kq + e.
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
        const uint32_t r = row0 + wr * (kRT * 16) + rt * 16 + r16;
        if (r >= p.rows) continue;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t t = cb * kColBlock + wc * 32 + ct * 16 + 4 * kq + e;
                if (t < p.n) p.y[size_t(t) * p.rows + r] = acc[rt][ct][e];
            }
    }
}

constexpr size_t wide_lds_bytes(int meta) {
    return 2 * size_t(kStageBytes) + 2 * 2 * size_t(kRowBlock) * kMetaGroups * (meta == 0 ? 4 : 2);
}

template <int META>
hipError_t launch_meta(const WideParams &p, hipStream_t stream) {
    auto kernel = wide_mfma_kernel<META>;
    constexpr size_t lds = wide_lds_bytes(META);
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess) return e;
        configured = true;
    }
    const uint32_t grid = (p.nrb + 7) / 8 * 8 * p.ncb;  // XCD-aware order; surplus workgroups exit
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kWideThreads), lds, stream, p);
    return hipGetLastError();
}

}  // namespace

bool wide_mfma_supported(const AffineArgs &a) {
    if (a.bits != 4 || a.group != 64) return false;
    if (a.meta != Meta::F32 && a.meta != Meta::BF16) return false;
    if (a.batch < 1 || a.batch > 256) return false;
    if (a.cols % (64 * kMetaGroups) != 0) return false;  // whole 8-group metadata copies
    const uintptr_t al = reinterpret_cast<uintptr_t>(a.w) | reinterpret_cast<uintptr_t>(a.s) |
                         reinterpret_cast<uintptr_t>(a.b);
    const uint64_t w_bytes = uint64_t(a.rows) * a.cols / 2;
    const uint64_t img = uint64_t(a.cols / 64) * ((a.batch + kColBlock - 1) / kColBlock) * kImgBytes;
    return al % 16 == 0 && uint64_t(a.batch) * a.cols * 4 < (1ull << 31) && w_bytes < (1ull << 31) &&
           img < (1ull << 31);
}

size_t wide_mfma_workspace(const AffineArgs &a) {
    const size_t ncb = (a.batch + kColBlock - 1) / kColBlock;
    return size_t(a.cols / 64) * ncb * kImgBytes;
}

hipError_t launch_wide_mfma(const AffineArgs &a, unsigned char *workspace, const DeviceLimits &lim,
                            hipStream_t stream) {
    const size_t lds = wide_lds_bytes(a.meta == Meta::F32 ? 0 : 1);
    if (lds > lim.max_lds_per_block) return hipErrorNotSupported;
    WideParams p;
    p.w = a.w;
    p.s = a.s;
    p.b = a.b;
    p.x = a.x;
    p.y = a.y;
    p.img = workspace;
    p.rows = a.rows;
    p.cols = a.cols;
    p.n = a.batch;
    p.ncb = (a.batch + kColBlock - 1) / kColBlock;
    p.nrb = (a.rows + kRowBlock - 1) / kRowBlock;
    p.w_bytes = uint32_t(uint64_t(a.rows) * a.cols / 2);
    p.m_bytes = uint32_t(uint64_t(a.rows) * (a.cols / 64) * (a.meta == Meta::F32 ? 4 : 2));
    p.img_bytes = uint32_t(wide_mfma_workspace(a));
    hipLaunchKernelGGL(wide_prep_kernel, dim3(a.cols / 64, p.ncb), dim3(kPrepThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return a.meta == Meta::F32 ? launch_meta<0>(p, stream) : launch_meta<1>(p, stream);
}

}  // namespace qmr

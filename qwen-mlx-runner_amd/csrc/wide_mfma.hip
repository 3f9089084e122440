// Wide block (chunked prefill) on the matrix cores: Q4/g64 weights times up
// to 256 RHS, y[t][r] = sum_c (q[r,c]*s[r,g] + b[r,g]) * x[t][c], computed
// in the factored form
//     y[t][r] = sum_g ( s[r,g] * D[r,t,g] + b[r,g] * S[t,g] ),
//     D[r,t,g] = sum_{c in g} q[r,c] * x[t,c],  S[t,g] = sum_{c in g} x[t,c].
// D runs on v_mfma_f32_16x16x32_f16 with exact integer codes (f16
// subnormals q*2^-20, as in mfma_common.hpp) against x split into hi/lo f16
// parts, so it is accurate to about 2^-22; the scales multiply D in FP32 and
// the bias term is an FP32 matrix product of S and b (v_mfma_f32_16x16x4_f32
// over four groups at a time).
//
// Two launches:
//   1. wide_prep_kernel turns x into one image per (quant group, block of 32
//      RHS): the group's eight MFMA A fragments (2 K steps x 2 RHS tiles x
//      hi/lo, 1 KB each, in lane order), the group sums S of the 32 RHS and
//      the factor 2^(20+e) of the block's power-of-two scale 2^-e.
//   2. wide_mfma_kernel: a workgroup of four waves (one per SIMD) owns
//      16*NRT rows x 32 RHS. Wave w takes every fourth quant group, g = w
//      (mod 4), so the four waves read the four 32-byte pieces of the same
//      128-byte code lines at about the same time (one L2 fetch, three L1
//      hits) and each x fragment is loaded once. A wave covers all row tiles
//      and both RHS tiles (8 FP32 accumulators per lane and row tile; a
//      second wave per SIMD gains nothing here, the vector ALU and the
//      matrix cores of a SIMD barely overlap). Per group it loads the 8 x
//      fragments (one group ahead) and one 8-byte code piece per row tile
//      (the next group's piece is requested as soon as this one is unpacked)
//      straight into registers. Scales (already multiplied by the image
//      factors) and biases stream through LDS in chunks of 16 groups, two
//      buffers, loaded by the whole workgroup one chunk ahead. At the end the
//      four group classes meet in LDS and are added in a fixed order.
// With NRT = 17 the 17408-row MLP matrix is 64 row blocks, which with four
// 32-RHS blocks at 128 RHS is one workgroup per CU of the 256.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <type_traits>
#include <vector>

#include "kernels.hpp"
#include "mfma_common.hpp"

namespace qmr {
namespace {

using namespace mfma;

typedef uint32_t u2 __attribute__((ext_vector_type(2)));

constexpr int kPrepThreads = 256;
constexpr int kKRanges = 4;                      // group classes (g mod 4) per workgroup
constexpr int kWaves = kKRanges;                  // one wave per group class
constexpr int kThreads = 64 * kWaves;
constexpr int kRhsBlock = 32;                     // RHS per workgroup and per image
constexpr int kFragBytes = 1024;                  // one MFMA A fragment (64 lanes x 16 B)
constexpr int kImgS = 8 * kFragBytes;             // S[32] f32
constexpr int kImgFac = kImgS + kRhsBlock * 4;    // factor f32
constexpr int kImgBytes = 8448;                   // image stride (16-byte multiple)
static_assert(kImgFac + 4 <= kImgBytes, "image layout");

// Metadata chunk in LDS (one of two buffers): s' (f32) and b (f32 for F32
// metadata, bf16 for BF16) of 16 groups, [row][group] with a pitch of 20
// entries (4 mod 8: the 16 rows one read touches fall in 16 banks).
constexpr int kCG = 16;  // groups per chunk: one quad per group class
constexpr int kPitch = 20;
template <int META>
constexpr size_t meta_buf_bytes(int nrt) {
    return size_t(16) * nrt * kPitch * (4 + (META == 0 ? 4 : 2));
}
template <int META>
constexpr size_t wide_lds_bytes(int nrt) {
    const size_t meta = 2 * meta_buf_bytes<META>(nrt);
    const size_t red = size_t(kKRanges) * nrt * 2 * 4 * 64 * 4;  // [class][rt][ct][v][lane] f32
    return meta > red ? meta : red;
}

// Byte offsets of the contraction kernel's code, x-fragment and group-sum
// loads, as the per-lane vector offset and the wave-uniform scalar offset of
// a buffer load. A load outside its view (a row past the matrix, a group
// past the row, an image past the last group) gets the vector offset kOut,
// which by itself lies past every view's extent, so it reads zeros whether
// or not the range check adds the scalar offset (kOut plus any scalar offset
// here stays below 2^32); every other load has voffset + soffset + size
// within its view. qmr_wide_address_extent walks every load the kernel can
// issue through these functions on the host.
struct WideAddr {
    uint32_t rows, G, ntb, row_bytes;
    // The 8-byte code piece of lane (r16, q) in row tile rt of the row block
    // at row0, quant group g (lanes q hold the group's four 16-column quarters).
    __host__ __device__ uint32_t code_v(uint32_t row0, uint32_t rt, uint32_t r16, uint32_t q, uint32_t g) const {
        return (row0 + 16 * rt + r16 < rows && g < G) ? (row0 + r16) * row_bytes + q * 8 : kOut;
    }
    __host__ __device__ uint32_t code_s(uint32_t rt, uint32_t g) const { return rt * 16 * row_bytes + g * 32; }
    // Fragment f of group g's image for RHS block tb; lane l reads 16 bytes.
    __host__ __device__ uint32_t frag_v(uint32_t lane, uint32_t g) const { return g < G ? lane * 16 : kOut; }
    __host__ __device__ uint32_t frag_s(uint32_t g, uint32_t tb, uint32_t f) const {
        return (g * ntb + tb) * uint32_t(kImgBytes) + f * uint32_t(kFragBytes);
    }
    // Group sum of RHS 16 ct + r16 in block tb for group g0 + 4 q (lane
    // (r16, q)); g0 = 16 c + class.
    __host__ __device__ uint32_t sum_v(uint32_t g0, uint32_t q, uint32_t r16, uint32_t ct) const {
        return g0 + 4 * q < G ? q * 4 * ntb * uint32_t(kImgBytes) + uint32_t(kImgS) + r16 * 4 + ct * 64 : kOut;
    }
    __host__ __device__ uint32_t sum_s(uint32_t g0, uint32_t tb) const {
        return (g0 * ntb + tb) * uint32_t(kImgBytes);
    }
};

struct WideParams {
    const uint32_t *w;
    const void *s;
    const void *b;
    const float *x;
    float *y;
    const unsigned char *img;  // [G][NTB] images of kImgBytes
    uint32_t rows, cols, n;    // n = RHS count
    uint32_t ntb;              // 32-RHS blocks
    uint32_t nrb;              // row blocks
    uint32_t w_bytes, m_bytes, img_bytes;  // extents of the views
};

// ---- 1. Activation images. grid (G, NTB), 256 threads: thread -> RHS
// tid/8 of the block and the 8 columns 8*(tid%8).. of the group, which is
// code word tid%8 of every row: K step tid%2, lane group tid/2 of the MFMA
// fragments. ----
__global__ __launch_bounds__(kPrepThreads) void wide_prep_kernel(WideParams p) {
    __shared__ float red[kPrepThreads / 64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const uint32_t g = blockIdx.x, tb = blockIdx.y;
    const uint32_t tt = uint32_t(tid) >> 3, c = uint32_t(tid) & 7;
    const uint32_t t = tb * kRhsBlock + tt;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(p.x), 0, int(p.n * p.cols * 4u), kRsrcWord3);
    float xv[8];
    load_x8(xv, xr, t, g * 64 + 8 * c, p.cols, t < p.n);
    float sum = 0.f, mx = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sum += xv[j];
        mx = fmaxf(mx, fabsf(xv[j]));
    }
    group_reduce<8>(sum, mx);  // one RHS: 8 consecutive lanes
    float m = mx;
#pragma unroll
    for (int o = 8; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
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
    unsigned char *img = const_cast<unsigned char *>(p.img) + (size_t(g) * p.ntb + tb) * kImgBytes;
    const uint32_t ks = c & 1, q = c >> 1, ct = tt >> 4;
    const uint32_t ln = q * 16 + (tt & 15);
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
        const float v0 = xv[k_of<4>(2 * e2)] * sc;
        const float v1 = xv[k_of<4>(2 * e2 + 1)] * sc;
        const h2 hh = __builtin_convertvector(f2{v0, v1}, h2);
        const h2 ll = __builtin_convertvector(f2{v0 - static_cast<float>(hh.x), v1 - static_cast<float>(hh.y)}, h2);
        hw[e2] = __builtin_bit_cast(uint32_t, hh);
        lw[e2] = __builtin_bit_cast(uint32_t, ll);
    }
    unsigned char *frag = img + ((ks * 2 + ct) * 2) * kFragBytes + ln * 16;
    *reinterpret_cast<u4 *>(frag) = u4{hw[0], hw[1], hw[2], hw[3]};
    *reinterpret_cast<u4 *>(frag + kFragBytes) = u4{lw[0], lw[1], lw[2], lw[3]};
    if (c == 0) reinterpret_cast<float *>(img + kImgS)[tt] = sum;
    if (tid == 0) reinterpret_cast<float *>(img + kImgFac)[0] = __uint_as_float(uint32_t(127 + kCodeExp<4> + e) << 23);
}

// One Q4 word (8 codes) as a B operand, in k_of order.
__device__ __forceinline__ h8 unpack_word(uint32_t wd) {
    const u4 c[1] = {u4{wd, 0u, 0u, 0u}};
    return unpack<4>(c, 0);
}

// ---- 2. The contraction. grid: row blocks (padded to a multiple of 8) x
// NTB, 256 threads. Lane (r16, q): row r16 of every row tile, K chunk q of
// every K step; D element v of a tile is RHS 4q + v of its 16-RHS tile. ----
template <int META, int NRT>
__global__ __launch_bounds__(kThreads, 1) void wide_mfma_kernel(WideParams p) {
    constexpr int ROWS = 16 * NRT;
    constexpr int BSZ = META == 0 ? 4 : 2;
    constexpr size_t BUF = meta_buf_bytes<META>(NRT);
    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x;
    const int kr = __builtin_amdgcn_readfirstlane(tid >> 6);  // the wave's group class (uniform)
    const int lane = tid & 63;
    const int r16 = lane & 15, q = lane >> 4;
    // XCD-aware order: workgroup i runs on XCD i % 8, so the NTB workgroups
    // of one row block (which read the same codes at about the same time)
    // share an XCD and its L2.
    const uint32_t xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
    const uint32_t tb = slot % p.ntb;
    const uint32_t rb = (slot / p.ntb) * 8 + xcd;
    if (rb >= p.nrb) return;
    const uint32_t row0 = rb * ROWS;
    const uint32_t G = p.cols / 64;
    const uint32_t nch = (G + kCG - 1) / kCG;
    const uint32_t row_bytes = p.cols / 2;
    const WideAddr A{p.rows, G, p.ntb, row_bytes};
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t *>(p.w), 0, int(p.w_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t ir = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char *>(p.img), 0, int(p.img_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.s), 0, int(p.m_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.b), 0, int(p.m_bytes), kRsrcWord3);
    const uint32_t m_pitch = G * BSZ;
    const f4 zero{0.f, 0.f, 0.f, 0.f};
    float *red = reinterpret_cast<float *>(lds);  // final reduction [class][row tile][ct][v][lane]

    // Metadata chunk c (groups 16c..16c+15) of all the workgroup's rows,
    // staged by every thread: item (row, j) = groups 16c+4j..16c+4j+3 of one
    // row; thread tid always has j = tid % 4, so it needs the image factors
    // of 4 groups only. Past the matrix (rows or groups) everything is zero.
    constexpr int ITEMS = ROWS * 4;
    constexpr int PER_T = (ITEMS + kThreads - 1) / kThreads;
    using Raw = std::conditional_t<META == 0, u4, u2>;
    struct MStage {
        Raw s[PER_T], b[PER_T];
        float fac[4];
    };
    const uint32_t mj = uint32_t(tid) & 3;
    auto meta_issue = [&](MStage &st, uint32_t c) {
        const uint32_t g4 = c * kCG + 4 * mj;  // first group of this thread's items
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t g = g4 + uint32_t(k);
            const uint32_t off = g < G ? (g * p.ntb + tb) * kImgBytes + kImgFac : kOut;
            st.fac[k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ir, int(off), 0, 0));
        }
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const uint32_t it = uint32_t(tid) + uint32_t(i) * kThreads;
            const uint32_t rl = it >> 2;
            const bool live = it < uint32_t(ITEMS) && row0 + rl < p.rows && g4 < G;
            const uint32_t moff = live ? (row0 + rl) * m_pitch + g4 * BSZ : kOut;
            if constexpr (META == 0) {
                st.s[i] = __builtin_amdgcn_raw_buffer_load_b128(sr, int(moff), 0, 0);
                st.b[i] = __builtin_amdgcn_raw_buffer_load_b128(br, int(moff), 0, 0);
            } else {
                st.s[i] = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(sr, int(moff), 0, 0));
                st.b[i] = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(br, int(moff), 0, 0));
            }
        }
    };
    auto meta_commit = [&](const MStage &st, uint32_t c) {
        unsigned char *buf = lds + (c & 1) * BUF;
        float *ms = reinterpret_cast<float *>(buf);
        unsigned char *mb = buf + size_t(ROWS) * kPitch * 4;
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const uint32_t it = uint32_t(tid) + uint32_t(i) * kThreads;
            const uint32_t rl = it >> 2;
            if (it < uint32_t(ITEMS)) {
                float sv[4];
                if constexpr (META == 0) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) sv[k] = __uint_as_float(st.s[i][k]);
                } else {
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        sv[2 * k] = __uint_as_float(st.s[i][k] << 16);
                        sv[2 * k + 1] = __uint_as_float(st.s[i][k] & 0xFFFF0000u);
                    }
                }
                *reinterpret_cast<float4 *>(ms + rl * kPitch + 4 * mj) =
                    float4{sv[0] * st.fac[0], sv[1] * st.fac[1], sv[2] * st.fac[2], sv[3] * st.fac[3]};
                *reinterpret_cast<Raw *>(mb + (rl * kPitch + 4 * mj) * BSZ) = st.b[i];
            }
        }
    };

    // The wave's share: all row tiles, groups kr, kr+4, ...
    {
        constexpr int NTW = NRT;
        // Code piece of row tile rt: words 2q, 2q+1 of the group for row
        // row0 + 16 rt + r16 (WideAddr: rows past the matrix and groups past
        // the row read zeros through the vector offset).
        u2 cw[NTW];
        auto load_codes = [&](int rt, uint32_t g) {
            cw[rt] = __builtin_bit_cast(
                u2, __builtin_amdgcn_raw_buffer_load_b64(wr, int(A.code_v(row0, uint32_t(rt), uint32_t(r16), uint32_t(q), g)),
                                                         int(A.code_s(uint32_t(rt), g)), 0));
        };
        // x fragments of group g: f = (ks*2 + ct)*2 + hl, lane i at 16 i
        // (past the last group: zeros).
        auto load_x = [&](h8 (&xf)[8], uint32_t g) {
            const int xo = int(A.frag_v(uint32_t(lane), g));
#pragma unroll
            for (int f = 0; f < 8; ++f)
                xf[f] = __builtin_bit_cast(
                    h8, __builtin_amdgcn_raw_buffer_load_b128(ir, xo, int(A.frag_s(g, tb, uint32_t(f))), 0));
        };
        // Bias A operands of chunk c: S[16c + 4q + kr][16 ct + r16].
        auto load_s = [&](float (&sop)[2], uint32_t c) {
            const uint32_t g0 = c * kCG + uint32_t(kr);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
                sop[ct] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    ir, int(A.sum_v(g0, uint32_t(q), uint32_t(r16), uint32_t(ct))), int(A.sum_s(g0, tb)), 0));
        };

        f4 acc[NTW][2];
        // One group (chunk buffer cb, class step i): codes of g in cw (their
        // successors, group g+4, requested as each piece is unpacked), x
        // fragments of g in xf. Software-pipelined by row tile: step rt
        // issues the 8 MFMAs of tile rt and, on the vector ALU, the epilogue
        // of tile rt-1 and the unpacking of tile rt+1; a scheduling barrier
        // keeps the steps apart, which bounds the live registers.
        auto group = [&](const h8 (&xf)[8], uint32_t g, const float *ms, int i) {
            const float *msw = ms + r16 * kPitch + 4 * i + kr;
            h8 bc[2][2];  // [tile parity][K step]
            f4 dp0 = zero, dp1 = zero;
            float svp = 0.f;
            bc[0][0] = unpack_word(cw[0].x);
            bc[0][1] = unpack_word(cw[0].y);
            load_codes(0, g + 4);
            float svn = msw[0];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int rt = 0; rt < NTW; ++rt) {
                const h8 b0 = bc[rt & 1][0], b1 = bc[rt & 1][1];
                f4 d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[0], b0, zero, 0, 0, 0);
                f4 d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[2], b0, zero, 0, 0, 0);
                d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[1], b0, d0, 0, 0, 0);
                d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[3], b0, d1, 0, 0, 0);
                d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[4], b1, d0, 0, 0, 0);
                d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[6], b1, d1, 0, 0, 0);
                d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[5], b1, d0, 0, 0, 0);
                d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[7], b1, d1, 0, 0, 0);
                if (rt > 0) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        acc[rt - 1][0][v] = __builtin_fmaf(svp, dp0[v], acc[rt - 1][0][v]);
                        acc[rt - 1][1][v] = __builtin_fmaf(svp, dp1[v], acc[rt - 1][1][v]);
                    }
                }
                if (rt + 1 < NTW) {
                    bc[(rt + 1) & 1][0] = unpack_word(cw[rt + 1].x);
                    bc[(rt + 1) & 1][1] = unpack_word(cw[rt + 1].y);
                    load_codes(rt + 1, g + 4);
                }
                svp = svn;
                if (rt + 1 < NTW) svn = msw[(rt + 1) * 16 * kPitch];
                dp0 = d0;
                dp1 = d1;
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                acc[NTW - 1][0][v] = __builtin_fmaf(svp, dp0[v], acc[NTW - 1][0][v]);
                acc[NTW - 1][1][v] = __builtin_fmaf(svp, dp1[v], acc[NTW - 1][1][v]);
            }
        };
        // Bias of the wave's four groups of a chunk: acc += S x b.
        auto bias = [&](const float (&sop)[2], const unsigned char *mb) {
#pragma unroll
            for (int rt = 0; rt < NTW; ++rt) {
                const uint32_t e = (rt * 16 + r16) * kPitch + 4 * q + kr;
                float bvv;
                if constexpr (META == 0)
                    bvv = reinterpret_cast<const float *>(mb)[e];
                else
                    bvv = __uint_as_float(uint32_t(reinterpret_cast<const uint16_t *>(mb)[e]) << 16);
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
                    acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(sop[ct], bvv, acc[rt][ct], 0, 0, 0);
            }
        };

        // All first requests in flight together (chunk 0's metadata, the
        // first group's codes and x, chunk 0's S), then chunk 0 into LDS.
        h8 xa[8], xb[8];
        float sa[2], sb[2];
        {
            MStage st;
            meta_issue(st, 0);
            load_x(xa, uint32_t(kr));
            load_s(sa, 0);
#pragma unroll
            for (int rt = 0; rt < NTW; ++rt) load_codes(rt, uint32_t(kr));
            __builtin_amdgcn_sched_barrier(0);  // every request before any use
            meta_commit(st, 0);
        }
#pragma unroll
        for (int rt = 0; rt < NTW; ++rt) acc[rt][0] = acc[rt][1] = zero;
        lds_barrier();
        // Chunk c: this wave's groups 16c + kr + 4i, i = 0..3. The next
        // chunk's metadata is requested first and committed to the other
        // buffer at the end (after the last chunk: zeros, never read), so the
        // loop body has no branch.
        for (uint32_t c = 0; c < nch; ++c) {
            const unsigned char *buf = lds + (c & 1) * BUF;
            const float *ms = reinterpret_cast<const float *>(buf);
            const unsigned char *mb = buf + size_t(ROWS) * kPitch * 4;
            const uint32_t g = c * kCG + uint32_t(kr);
            MStage st;
            meta_issue(st, c + 1);
            load_s(sb, c + 1);
            load_x(xb, g + 4);
            group(xa, g, ms, 0);
            load_x(xa, g + 8);
            group(xb, g + 4, ms, 1);
            load_x(xb, g + 12);
            group(xa, g + 8, ms, 2);
            load_x(xa, g + 16);
            group(xb, g + 12, ms, 3);
            bias(sa, mb);
            sa[0] = sb[0];
            sa[1] = sb[1];
            meta_commit(st, c + 1);
            lds_barrier();
        }

        // The group classes meet in LDS (the metadata buffers are free).
#pragma unroll
        for (int rt = 0; rt < NTW; ++rt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    red[(((kr * NRT + rt) * 2 + ct) * 4 + v) * 64 + lane] = acc[rt][ct][v];
    }
    lds_barrier();
    // Wave w writes the (row tile, ct, v) combinations w, w+4, ...: lane
    // (r16, q) holds row 16 rt + r16 and RHS 16 ct + 4 q + v; the four group
    // classes are added in order.
    for (int cmb = kr; cmb < NRT * 8; cmb += kWaves) {
        float sum = 0.f;
#pragma unroll
        for (int k = 0; k < kKRanges; ++k) sum += red[(k * NRT * 8 + cmb) * 64 + lane];
        const uint32_t rt = uint32_t(cmb) >> 3, ct = (uint32_t(cmb) >> 2) & 1, v = uint32_t(cmb) & 3;
        const uint32_t r = row0 + rt * 16 + uint32_t(r16);
        const uint32_t t = tb * kRhsBlock + ct * 16 + uint32_t(q) * 4 + v;
        if (r < p.rows && t < p.n) p.y[size_t(t) * p.rows + r] = sum;
    }
}

// Resident workgroups per CU of a kernel instance (as the runtime computes
// it from registers and LDS); cached.
uint32_t resident_per_cu(const void *kernel, size_t lds) {
    struct Entry {
        const void *k;
        size_t lds;
        uint32_t n;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry &e : cache)
        if (e.k == kernel && e.lds == lds) return e.n;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kThreads, lds) != hipSuccess || n < 1) n = 1;
    cache.push_back(Entry{kernel, lds, uint32_t(n)});
    return uint32_t(n);
}

template <int META, int NRT>
hipError_t launch_nrt(WideParams p, hipStream_t stream) {
    auto kernel = wide_mfma_kernel<META, NRT>;
    constexpr size_t lds = wide_lds_bytes<META>(NRT);
    {
        const hipError_t e = raise_lds_limit(reinterpret_cast<const void *>(kernel), lds);
        if (e != hipSuccess) return e;
    }
    p.nrb = (p.rows + 16 * NRT - 1) / (16 * NRT);
    const uint32_t grid = (p.nrb + 7) / 8 * 8 * p.ntb;  // XCD-aware order; surplus workgroups exit
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), lds, stream, p);
    return hipGetLastError();
}

// Rounds of resident workgroups times rows per workgroup: the planner's cost
// of a row-tile count (the work of one round grows with NRT).
template <int META, int NRT>
double wide_cost(const WideParams &p, const DeviceLimits &lim) {
    const uint32_t nrb = (p.rows + 16 * NRT - 1) / (16 * NRT);
    const uint32_t per_cu = resident_per_cu(reinterpret_cast<const void *>(wide_mfma_kernel<META, NRT>),
                                            wide_lds_bytes<META>(NRT));
    const uint32_t slots = per_cu * uint32_t(std::max(lim.num_cus, 1));
    const uint32_t wgs = nrb * p.ntb;
    return double((wgs + slots - 1) / slots) * NRT * per_cu;
}

template <int META>
hipError_t launch_meta(const WideParams &p, const DeviceLimits &lim, hipStream_t stream) {
    if (wide_lds_bytes<META>(17) <= lim.max_lds_per_block && wide_cost<META, 17>(p, lim) <= wide_cost<META, 8>(p, lim))
        return launch_nrt<META, 17>(p, stream);
    if (wide_lds_bytes<META>(8) > lim.max_lds_per_block) return hipErrorNotSupported;
    return launch_nrt<META, 8>(p, stream);
}

}  // namespace

bool wide_mfma_supported(const AffineArgs &a) {
    if (a.bits != 4 || a.group != 64) return false;
    if (a.meta != Meta::F32 && a.meta != Meta::BF16) return false;
    if (a.batch < 1 || a.batch > 256) return false;
    if (a.cols % 256 != 0) return false;  // whole quads of groups (metadata items)
    const uintptr_t al = reinterpret_cast<uintptr_t>(a.w) | reinterpret_cast<uintptr_t>(a.s) |
                         reinterpret_cast<uintptr_t>(a.b);
    // 32-bit buffer offsets: codes reach one workgroup's rows plus a row
    // past the matrix, images and prefetches up to a chunk plus a quad of
    // groups past the last one (all read as zeros).
    const uint64_t w_span = (uint64_t(a.rows) + 16 * 17 + 2) * a.cols / 2;
    const uint64_t ntb = (a.batch + kRhsBlock - 1) / kRhsBlock;
    const uint64_t img = (uint64_t(a.cols / 64) + kCG + 8) * ntb * kImgBytes;
    return al % 16 == 0 && uint64_t(a.batch) * a.cols * 4 < (1ull << 31) && w_span < (1ull << 31) &&
           img < (1ull << 31);
}

size_t wide_mfma_workspace(const AffineArgs &a) {
    const size_t ntb = (a.batch + kRhsBlock - 1) / kRhsBlock;
    return size_t(a.cols / 64) * ntb * kImgBytes;
}

WideExtent wide_address_extent(uint32_t rows, uint32_t cols, uint32_t n, uint32_t nrt) {
    WideExtent out{};
    const uint32_t G = cols / 64, nch = (G + kCG - 1) / kCG, ntb = (n + kRhsBlock - 1) / kRhsBlock;
    const uint32_t nrb = (rows + 16 * nrt - 1) / (16 * nrt);
    const WideAddr A{rows, G, ntb, cols / 2};
    out.code_extent = uint64_t(rows) * cols / 2;
    out.image_extent = uint64_t(G) * ntb * kImgBytes;
    auto note = [](uint64_t &mx, uint32_t v, uint32_t so, uint32_t size) {
        if (v != kOut) mx = std::max(mx, uint64_t(v) + so + size);
    };
    // Groups the kernel requests per class kr: the first (kr) and, for each
    // group it processes (16c + kr + 4i, c < nch, i < 4), the one four
    // groups on (codes and x fragments alike); group sums per chunk c <= nch.
    for (uint32_t kr = 0; kr < uint32_t(kKRanges); ++kr) {
        for (uint32_t j = 0; j <= 4 * nch; ++j) {
            const uint32_t g = kr + 4 * j;
            for (uint32_t rb = 0; rb < nrb; ++rb)
                for (uint32_t rt = 0; rt < nrt; ++rt)
                    for (uint32_t l = 0; l < 64; ++l)
                        note(out.code_end, A.code_v(rb * 16 * nrt, rt, l & 15, l >> 4, g), A.code_s(rt, g), 8);
            for (uint32_t tb = 0; tb < ntb; ++tb)
                for (uint32_t f = 0; f < 8; ++f)
                    for (uint32_t l = 0; l < 64; ++l) note(out.image_end, A.frag_v(l, g), A.frag_s(g, tb, f), 16);
        }
        for (uint32_t c = 0; c <= nch; ++c)
            for (uint32_t tb = 0; tb < ntb; ++tb)
                for (uint32_t l = 0; l < 64; ++l)
                    for (uint32_t ct = 0; ct < 2; ++ct)
                        note(out.image_end, A.sum_v(c * kCG + kr, l >> 4, l & 15, ct), A.sum_s(c * kCG + kr, tb), 4);
    }
    return out;
}

hipError_t launch_wide_mfma(const AffineArgs &a, unsigned char *workspace, const DeviceLimits &lim,
                            hipStream_t stream) {
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
    p.ntb = (a.batch + kRhsBlock - 1) / kRhsBlock;
    p.nrb = 0;
    p.w_bytes = uint32_t(uint64_t(a.rows) * a.cols / 2);
    p.m_bytes = uint32_t(uint64_t(a.rows) * (a.cols / 64) * (a.meta == Meta::F32 ? 4 : 2));
    p.img_bytes = uint32_t(wide_mfma_workspace(a));
    hipLaunchKernelGGL(wide_prep_kernel, dim3(a.cols / 64, p.ntb), dim3(kPrepThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return a.meta == Meta::F32 ? launch_meta<0>(p, lim, stream) : launch_meta<1>(p, lim, stream);
}

}  // namespace qmr

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
//   2. wide_mfma_kernel: a workgroup of eight waves owns 16*NRT rows x 32
//      RHS. K is split into four ranges of whole quads of groups and the row
//      tiles into two halves; wave w takes K range w%4 and half w/4, so the
//      two waves sharing a SIMD have the same instruction mix and one's
//      matrix-core work overlaps the other's vector-ALU work. A wave covers
//      both RHS tiles of its row tiles (8 FP32 accumulators per lane and row
//      tile). Per group it loads the 8 x fragments (one group ahead) and one
//      8-byte code piece per row tile (the next group's piece is requested as
//      soon as this one is unpacked) straight into registers. Scales (already
//      multiplied by the image factors) and biases of the wave's rows and K
//      range go through LDS, staged by the wave itself. At the end the four
//      K ranges meet in LDS and are added in K order.
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
constexpr int kKRanges = 4;                      // K ranges per workgroup
constexpr int kFirstHalf17 = 10;                  // row tiles of the first half at NRT = 17
constexpr int kWaves = 2 * kKRanges;              // two row halves per K range
constexpr int kThreads = 64 * kWaves;
constexpr int kRhsBlock = 32;                     // RHS per workgroup and per image
constexpr int kFragBytes = 1024;                  // one MFMA A fragment (64 lanes x 16 B)
constexpr int kImgS = 8 * kFragBytes;             // S[32] f32
constexpr int kImgFac = kImgS + kRhsBlock * 4;    // factor f32
constexpr int kImgBytes = 8448;                   // image stride (16-byte multiple)
static_assert(kImgFac + 4 <= kImgBytes, "image layout");

// Metadata staged per wave and chunk of groups: s' (f32) and b (f32 for F32
// metadata, bf16 for BF16), [row][group] with a pitch of CG entries; CG is a
// multiple of 4 that is 4 mod 8, so the 16 rows one read touches fall in 16
// different banks.
template <int META>
struct MetaCfg {
    static constexpr int CG = META == 0 ? 12 : 20;  // groups per chunk
    static constexpr int BSZ = META == 0 ? 4 : 2;   // bytes of a staged bias
    static_assert(CG % 8 == 4, "pitch");
};

template <int META>
constexpr size_t wave_meta_bytes(int nrt) {
    return size_t(16) * nrt * MetaCfg<META>::CG * (4 + MetaCfg<META>::BSZ);
}
// Row tiles of the first row half (waves 0-3). The hardware issues the
// older of two waves sharing a SIMD first, so the first half gets the larger
// share of the row tiles and both halves finish at about the same time.
constexpr int first_half_tiles(int nrt) { return nrt == 17 ? kFirstHalf17 : (nrt + 1) / 2; }
template <int META>
constexpr size_t wide_lds_bytes(int nrt) {
    const size_t meta = kKRanges * (wave_meta_bytes<META>(first_half_tiles(nrt)) +
                                    wave_meta_bytes<META>(nrt - first_half_tiles(nrt))) +
                        kWaves * MetaCfg<META>::CG * 4;
    const size_t red = size_t(kKRanges) * nrt * 2 * 4 * 64 * 4;  // [K range][rt][ct][v][lane] f32
    return meta > red ? meta : red;
}

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
// NTB, 512 threads. Wave w takes K range w%4 and row half w/4 (the first
// ceil(NRT/2) row tiles or the rest); the two waves of a K range share a
// SIMD, so one's matrix-core work overlaps the other's vector-ALU work.
// Lane (r16, q): row r16 of every row tile, K chunk q of every K step; D
// element v of a tile is RHS 4q + v of its 16-RHS tile. ----
template <int META, int NRT>
__global__ __launch_bounds__(kThreads, 1) void wide_mfma_kernel(WideParams p) {
    using MC = MetaCfg<META>;
    constexpr int CG = MC::CG;
    constexpr int CQ = CG / 4;  // quads per chunk
    constexpr int NRT0 = first_half_tiles(NRT);
    constexpr int MR0 = int(wave_meta_bytes<META>(NRT0)), MR1 = int(wave_meta_bytes<META>(NRT - NRT0));
    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: K range, rows, LDS regions
    const int kr = wave & 3, rh = wave >> 2;
    const int lane = tid & 63;
    const int r16 = lane & 15, q = lane >> 4;
    // XCD-aware order: workgroup i runs on XCD i % 8, so the NTB workgroups
    // of one row block (which read the same codes at about the same time)
    // share an XCD and its L2.
    const uint32_t xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
    const uint32_t tb = slot % p.ntb;
    const uint32_t rb = (slot / p.ntb) * 8 + xcd;
    if (rb >= p.nrb) return;
    const uint32_t row0 = rb * 16 * NRT;
    const uint32_t G = p.cols / 64;
    const uint32_t nq = G / 4;
    const uint32_t qa = uint32_t(kr) * nq / kKRanges, qb = uint32_t(kr + 1) * nq / kKRanges;
    const uint32_t ga = qa * 4, gb = qb * 4;  // this wave's groups [ga, gb)
    const uint32_t row_bytes = p.cols / 2;
    const int rtb = rh ? NRT0 : 0;  // first row tile of this wave
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t *>(p.w), 0, int(p.w_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t ir = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char *>(p.img), 0, int(p.img_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.s), 0, int(p.m_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.b), 0, int(p.m_bytes), kRsrcWord3);
    const uint32_t m_pitch = G * (META == 0 ? 4 : 2);
    const f4 zero{0.f, 0.f, 0.f, 0.f};
    float *red = reinterpret_cast<float *>(lds);  // final reduction [kr][row tile][ct][v][lane]

    // The wave's share: NTW row tiles from rtb, K range [ga, gb).
    auto run = [&](auto ntw_c) {
        constexpr int NTW = decltype(ntw_c)::value;
        const uint32_t wrow0 = row0 + uint32_t(rtb) * 16;
        // Code piece of row tile rt: words 2q, 2q+1 of the group for row
        // wrow0 + 16 rt + r16. The row tile and group move only the scalar
        // offset; the buffer range check covers vector plus scalar offset,
        // so rows past the matrix read zeros.
        const uint32_t cbase = (wrow0 + uint32_t(r16)) * row_bytes + uint32_t(q) * 8;
        const uint32_t cstride = 16 * row_bytes;
        u2 cw[NTW];
        auto load_codes = [&](int rt, uint32_t g) {
            cw[rt] = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(
                                                 wr, int(cbase), int(uint32_t(rt) * cstride + g * 32), 0));
        };
        // x fragments of group g: f = (ks*2 + ct)*2 + hl, lane i at 16 i.
        const uint32_t xo = uint32_t(lane) * 16;
        auto load_x = [&](h8 (&xf)[8], uint32_t g) {
            const int base = int((g * p.ntb + tb) * kImgBytes);
#pragma unroll
            for (int f = 0; f < 8; ++f)
                xf[f] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(ir, int(xo), base + f * kFragBytes, 0));
        };
        // Bias A operands of the quad at group g0: S[g0 + q][16 ct + r16].
        const uint32_t so = uint32_t(q) * p.ntb * kImgBytes + kImgS + uint32_t(r16) * 4;
        auto load_s = [&](float (&sop)[2], uint32_t g0) {
            const int base = int((g0 * p.ntb + tb) * kImgBytes);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
                sop[ct] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ir, int(so + ct * 64), base, 0));
        };

        // Metadata chunk staging (this wave's region; only this wave reads
        // it): every load of a chunk is issued first (meta_issue), the
        // conversion and LDS writes follow (meta_commit).
        unsigned char *wm = lds + (rh ? size_t(kKRanges) * MR0 + size_t(kr) * MR1 : size_t(kr) * MR0);
        float *ms = reinterpret_cast<float *>(wm);                  // s' [NTW*16][CG]
        unsigned char *mbias = wm + size_t(NTW) * 16 * CG * 4;      // b  [NTW*16][CG]
        float *mfac = reinterpret_cast<float *>(lds + size_t(kKRanges) * (MR0 + MR1)) + wave * CG;
        constexpr int ITEMS = NTW * 16 * CQ;  // (row, quad): 4 groups of s and b of one row
        constexpr int PER_LANE = (ITEMS + 63) / 64;
        using Raw = std::conditional_t<META == 0, u4, u2>;
        struct Staged {
            Raw s[PER_LANE], b[PER_LANE];
            float fac;  // factor of group gc0 + lane (lanes < CG)
        };
        auto meta_issue = [&](Staged &st, uint32_t gc0, uint32_t ngc) {
            const uint32_t foff = uint32_t(lane) < ngc ? ((gc0 + uint32_t(lane)) * p.ntb + tb) * kImgBytes + kImgFac : kOut;
            st.fac = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ir, int(foff), 0, 0));
            const uint32_t nqc = ngc / 4;
#pragma unroll
            for (int i = 0; i < PER_LANE; ++i) {
                const uint32_t it = uint32_t(lane) + uint32_t(i) * 64;
                const uint32_t rl = it / CQ, j = it - rl * CQ;
                const bool live = it < uint32_t(ITEMS) && j < nqc && wrow0 + rl < p.rows;
                const uint32_t moff = live ? (wrow0 + rl) * m_pitch + (gc0 + 4 * j) * (META == 0 ? 4 : 2) : kOut;
                if constexpr (META == 0) {
                    st.s[i] = __builtin_amdgcn_raw_buffer_load_b128(sr, int(moff), 0, 0);
                    st.b[i] = __builtin_amdgcn_raw_buffer_load_b128(br, int(moff), 0, 0);
                } else {
                    st.s[i] = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(sr, int(moff), 0, 0));
                    st.b[i] = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(br, int(moff), 0, 0));
                }
            }
        };
        auto meta_commit = [&](const Staged &st) {
            if (lane < CG) mfac[lane] = st.fac;
            wave_lds_sync();
#pragma unroll
            for (int i = 0; i < PER_LANE; ++i) {
                const uint32_t it = uint32_t(lane) + uint32_t(i) * 64;
                const uint32_t rl = it / CQ, j = it - rl * CQ;
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
                    const float4 fac = *reinterpret_cast<const float4 *>(mfac + 4 * j);
                    *reinterpret_cast<float4 *>(ms + rl * CG + 4 * j) =
                        float4{sv[0] * fac.x, sv[1] * fac.y, sv[2] * fac.z, sv[3] * fac.w};
                    if constexpr (META == 0)
                        *reinterpret_cast<u4 *>(mbias + (rl * CG + 4 * j) * 4) = st.b[i];
                    else
                        *reinterpret_cast<u2 *>(mbias + (rl * CG + 4 * j) * 2) = st.b[i];
                }
            }
            wave_lds_sync();
        };

        f4 acc[NTW][2];
        // One group: codes of g in cw (their g+1 successors requested as
        // each piece is unpacked), x fragments of g in xf. Software-pipelined
        // by row tile: step rt issues the 8 MFMAs of tile rt and, on the
        // vector ALU, the epilogue of tile rt-1 and the unpacking of tile
        // rt+1; a scheduling barrier keeps the steps apart, which bounds the
        // live registers.
        auto group = [&](const h8 (&xf)[8], uint32_t g, uint32_t gl) {
            const uint32_t gn = min(g + 1, gb - 1);  // last group: a harmless reload
            h8 bc[2][2];                               // [tile parity][K step]
            f4 dp0 = zero, dp1 = zero;
            float svp = 0.f;
            bc[0][0] = unpack_word(cw[0].x);
            bc[0][1] = unpack_word(cw[0].y);
            load_codes(0, gn);
            float svn = ms[r16 * CG + gl];
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
                    load_codes(rt + 1, gn);
                }
                svp = svn;
                if (rt + 1 < NTW) svn = ms[((rt + 1) * 16 + r16) * CG + gl];
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
        // Bias of the quad at chunk-local group gl0: acc += S x b over 4 groups.
        auto bias = [&](const float (&sop)[2], uint32_t gl0) {
#pragma unroll
            for (int rt = 0; rt < NTW; ++rt) {
                const uint32_t e = (rt * 16 + r16) * CG + gl0 + q;
                float bvv;
                if constexpr (META == 0)
                    bvv = reinterpret_cast<const float *>(mbias)[e];
                else
                    bvv = __uint_as_float(uint32_t(reinterpret_cast<const uint16_t *>(mbias)[e]) << 16);
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
                    acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(sop[ct], bvv, acc[rt][ct], 0, 0, 0);
            }
        };

        if (ga < gb) {
            // All first requests in flight together: the first chunk's
            // metadata, then the first group's codes and x and the first
            // quad's S; the metadata commit then waits for its own loads only.
            h8 xa[8], xb[8];
            float sa[2], sb[2];
            {
                Staged st;
                meta_issue(st, ga, min(uint32_t(CG), gb - ga));
                load_x(xa, ga);
                load_s(sa, ga);
#pragma unroll
                for (int rt = 0; rt < NTW; ++rt) load_codes(rt, ga);
                __builtin_amdgcn_sched_barrier(0);  // every request before any use
                meta_commit(st);
            }
#pragma unroll
            for (int rt = 0; rt < NTW; ++rt) acc[rt][0] = acc[rt][1] = zero;
            for (uint32_t gc0 = ga; gc0 < gb; gc0 += CG) {
                const uint32_t ngc = min(uint32_t(CG), gb - gc0);
                if (gc0 != ga) {
                    Staged st;
                    meta_issue(st, gc0, ngc);
                    meta_commit(st);
                }
                for (uint32_t gl = 0; gl < ngc; gl += 4) {
                    const uint32_t g = gc0 + gl;
                    load_s(sb, min(g + 4, gb - 4));  // next quad (last: a harmless reload)
                    load_x(xb, g + 1);
                    group(xa, g, gl);
                    load_x(xa, g + 2);
                    group(xb, g + 1, gl + 1);
                    load_x(xb, g + 3);
                    group(xa, g + 2, gl + 2);
                    load_x(xa, min(g + 4, gb - 1));  // last quad: a harmless reload
                    group(xb, g + 3, gl + 3);
                    bias(sa, gl);
                    sa[0] = sb[0];
                    sa[1] = sb[1];
                }
                wave_lds_sync();  // this chunk's metadata reads precede the next chunk's writes
            }
        } else {
#pragma unroll
            for (int rt = 0; rt < NTW; ++rt) acc[rt][0] = acc[rt][1] = zero;
        }

        // The K ranges meet in LDS once every wave is done with its
        // metadata region.
        lds_barrier();
#pragma unroll
        for (int rt = 0; rt < NTW; ++rt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    red[(((kr * NRT + rtb + rt) * 2 + ct) * 4 + v) * 64 + lane] = acc[rt][ct][v];
    };
    if (rh == 0)
        run(std::integral_constant<int, NRT0>{});
    else
        run(std::integral_constant<int, NRT - NRT0>{});
    lds_barrier();
    // Wave w writes the (row tile, ct, v) combinations w, w+8, ...: lane
    // (r16, q) holds row 16 rt + r16 and RHS 16 ct + 4 q + v; the four K
    // ranges are added in order.
    for (int cmb = wave; cmb < NRT * 8; cmb += kWaves) {
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
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess) return e;
        configured = true;
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
    if (a.cols % 256 != 0) return false;  // whole quads of groups
    const uintptr_t al = reinterpret_cast<uintptr_t>(a.w) | reinterpret_cast<uintptr_t>(a.s) |
                         reinterpret_cast<uintptr_t>(a.b);
    // Code offsets reach one workgroup's rows past the matrix.
    const uint64_t w_span = (uint64_t(a.rows) + 16 * 17) * a.cols / 2;
    const uint64_t img = uint64_t(a.cols / 64) * ((a.batch + kRhsBlock - 1) / kRhsBlock) * kImgBytes;
    return al % 16 == 0 && uint64_t(a.batch) * a.cols * 4 < (1ull << 31) && w_span < (1ull << 31) &&
           img < (1ull << 31);
}

size_t wide_mfma_workspace(const AffineArgs &a) {
    const size_t ntb = (a.batch + kRhsBlock - 1) / kRhsBlock;
    return size_t(a.cols / 64) * ntb * kImgBytes;
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

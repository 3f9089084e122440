// The rest of the reference's matrix dispatch surface:
//   - a reference-arithmetic affine GEMV/block for any group size (the
//     reference's generic matvec_affine, kernels/qwen.metal:40-68, which its
//     reference mode and unusual group sizes use);
//   - row dequantisation (embed_affine[_bf16], kernels/qwen.metal:73-77,
//     kernels/affine_bf16.metal:162-174), bit-exact RN32(q*s + b);
//   - dense F16 matvec / blocks / embedding (kernels/qwen.metal:48-57,69-72,
//     kernels/matmul_block.metal:213-248);
//   - copy_f32 (kernels/matmul_block.metal:315-318), a streaming copy that is
//     also the known-size kernel HBM byte counters are calibrated against;
//   - read_checksum (no reference counterpart): one pure streaming read of up
//     to three views, the read floor of a product's codes and metadata;
//   - a zero fill for workspace that must start cleared.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.hpp"
#include "mfma_common.hpp"

namespace qmr {
namespace {

__device__ __forceinline__ float meta_at(const void *p, size_t i, int meta) {
    if (meta == 0) return static_cast<const float *>(p)[i];
    const uint16_t h = static_cast<const uint16_t *>(p)[i];
    if (meta == 1) return __uint_as_float(uint32_t(h) << 16);
    return float(__builtin_bit_cast(_Float16, h));
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over all 64 lanes; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
    v += __shfl_xor(v, 32);
    return v;
}

// One wave per (row, rhs); lanes stride over columns. Per element the weight
// is dequantised first, w = float(q)*s + b, then multiplied by x: the order
// of the reference's affine() (kernels/qwen.metal:40-47).
__global__ __launch_bounds__(256) void affine_generic_kernel(
    const uint32_t *__restrict__ w, const void *__restrict__ s, const void *__restrict__ b,
    int meta, const float *__restrict__ x, float *__restrict__ y, uint32_t rows, uint32_t cols,
    uint32_t bits, uint32_t group, uint32_t batch) {
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t lane = threadIdx.x & 63;
    if (wave >= rows * batch) return;  // wave-uniform
    const uint32_t row = wave % rows, t = wave / rows;
    const uint32_t pack = 32 / bits, mask = (1u << bits) - 1u;
    const uint32_t *wr = w + size_t(row) * (cols / pack);
    const size_t gbase = size_t(row) * (cols / group);
    const float *xt = x + size_t(t) * cols;
    float v = 0.f;
    for (uint32_t c = lane; c < cols; c += 64) {
        const uint32_t q = (wr[c / pack] >> ((c % pack) * bits)) & mask;
        const size_t gi = gbase + c / group;
        const float wv = float(q) * meta_at(s, gi, meta) + meta_at(b, gi, meta);
        v += wv * xt[c];
    }
    v = wave_sum(v);
    if (lane == 0) y[size_t(t) * rows + row] = v;
}

// y[c] = RN32(RN32(q*s) + b), the reference's float(q) * s + b with each
// operation rounded (kernels/qwen.metal:40-47,73-77). With BF16 or F16
// metadata q*s is exact (at most 8 + 11 significant bits), so this equals
// RN32(q*s + b); with FP32 metadata the product is rounded first, so no
// fused multiply-add is used.
__global__ __launch_bounds__(256) void embed_affine_kernel(
    const uint32_t *__restrict__ w, const void *__restrict__ s, const void *__restrict__ b,
    int meta, uint32_t row, uint32_t cols, uint32_t bits, uint32_t group, float *__restrict__ y) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= cols) return;
    const uint32_t pack = 32 / bits;
    const uint32_t word = w[size_t(row) * (cols / pack) + c / pack];
    const uint32_t q = (word >> ((c % pack) * bits)) & ((1u << bits) - 1u);
    const size_t gi = size_t(row) * (cols / group) + c / group;
    {
#pragma clang fp contract(off)
        const float prod = float(q) * meta_at(s, gi, meta);
        y[c] = prod + meta_at(b, gi, meta);
    }
}

// Dense F16 weights times token-major FP32 x; one wave per (row, rhs).
__global__ __launch_bounds__(256) void dense_f16_kernel(const uint16_t *__restrict__ w,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, uint32_t rows,
                                                        uint32_t cols, uint32_t batch) {
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t lane = threadIdx.x & 63;
    if (wave >= rows * batch) return;
    const uint32_t row = wave % rows, t = wave / rows;
    const uint16_t *wr = w + size_t(row) * cols;
    const float *xt = x + size_t(t) * cols;
    float v = 0.f;
    for (uint32_t c = lane; c < cols; c += 64)
        v = __builtin_fmaf(float(__builtin_bit_cast(_Float16, wr[c])), xt[c], v);
    v = wave_sum(v);
    if (lane == 0) y[size_t(t) * rows + row] = v;
}

// Dense F16 weights times token-major FP32 x, streaming form for cols % 8 == 0
// and matrices under 2 GB: each lane takes 8 consecutive columns per
// 512-column step as one 16-byte weight load per row (buffer loads; rows past
// the matrix read as zeros). The x slice of a step is loaded once and used
// for the wave's R rows, and every RHS uses the same weight registers, so the
// matrix is read once whatever B. Two steps are requested before the first
// is used. KS = 1: each of the workgroup's four waves owns R rows for all of
// K. KS = 4: the four waves share R rows, wave k taking steps k, k + 4, ...;
// their sums meet in LDS and are added in wave order, so results do not
// depend on timing.
template <int B, int R, int KS>
__global__ __launch_bounds__(256) void dense_f16_stream_kernel(const uint16_t *__restrict__ w,
                                                               const float *__restrict__ x,
                                                               float *__restrict__ y, uint32_t rows,
                                                               uint32_t cols, uint32_t w_bytes) {
    static_assert(KS == 1 || KS == 4, "one wave per row group, or the workgroup's four");
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t row0 = KS == 1 ? (blockIdx.x * 4u + wave) * R : blockIdx.x * R;
    const uint32_t lane = threadIdx.x & 63;
    if (KS == 1 && row0 >= rows) return;  // the whole wave (KS = 4: the grid covers rows exactly)
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(w), 0, int(w_bytes), mfma::kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(x), 0, int(uint32_t(B) * cols * 4u), mfma::kRsrcWord3);
    float acc[R][B];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
        for (int t = 0; t < B; ++t) acc[i][t] = 0.f;
    auto load_w = [&](v4u (&wv)[R], uint32_t c) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const uint32_t off = (c < cols && row0 + i < rows) ? ((row0 + i) * cols + c) * 2u : mfma::kOut;
            wv[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, int(off), 0, 0);
        }
    };
    auto use = [&](const v4u (&wv)[R], uint32_t c) {
#pragma unroll
        for (int t = 0; t < B; ++t) {
            const uint32_t xo = c < cols ? (uint32_t(t) * cols + c) * 4u : mfma::kOut;
            const v4u xa = __builtin_amdgcn_raw_buffer_load_b128(xr, int(xo), 0, 0);
            const v4u xb = __builtin_amdgcn_raw_buffer_load_b128(xr, int(xo + 16u), 0, 0);
            float xv[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xv[j] = __uint_as_float(xa[j]);
                xv[4 + j] = __uint_as_float(xb[j]);
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // Through a scalar: a bit cast of the vector element
                    // itself reads the vector's first dword.
                    const uint32_t d = wv[i][j];
                    const h2v h = __builtin_bit_cast(h2v, d);
                    acc[i][t] = __builtin_fmaf(float(h.x), xv[2 * j], acc[i][t]);
                    acc[i][t] = __builtin_fmaf(float(h.y), xv[2 * j + 1], acc[i][t]);
                }
            }
        }
    };
    const uint32_t steps = (cols + 511) / 512;
    const uint32_t first = KS == 1 ? 0u : wave;
    constexpr uint32_t STRIDE = 512u * KS;  // columns between a wave's steps
    v4u w0[R], w1[R];
    load_w(w0, first * 512u + lane * 8u);
    for (uint32_t st = first; st < steps; st += 2 * KS) {
        const uint32_t c0 = st * 512u + lane * 8u;
        load_w(w1, c0 + STRIDE);
        use(w0, c0);
        load_w(w0, c0 + 2 * STRIDE);
        use(w1, c0 + STRIDE);
    }
    if constexpr (KS == 1) {
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int t = 0; t < B; ++t) {
                const float v = wave_sum(acc[i][t]);
                if (lane == 0 && row0 + i < rows) y[size_t(t) * rows + row0 + i] = v;
            }
    } else {
        __shared__ float part[KS][R][B];
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int t = 0; t < B; ++t) {
                const float v = wave_sum(acc[i][t]);
                if (lane == 0) part[wave][i][t] = v;
            }
        __syncthreads();
        if (threadIdx.x < uint32_t(R * B)) {
            const uint32_t i = threadIdx.x / B, t = threadIdx.x % B;
            float v = part[0][i][t];
#pragma unroll
            for (int k = 1; k < KS; ++k) v += part[k][i][t];
            if (row0 + i < rows) y[size_t(t) * rows + row0 + i] = v;
        }
    }
}

__global__ __launch_bounds__(256) void embed_f16_kernel(const uint16_t *__restrict__ w,
                                                        uint32_t row, uint32_t cols,
                                                        float *__restrict__ y) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c < cols) y[c] = float(__builtin_bit_cast(_Float16, w[size_t(row) * cols + c]));
}

}  // namespace

hipError_t launch_affine_generic(const AffineArgs &a, hipStream_t stream) {
    const uint64_t waves = uint64_t(a.rows) * a.batch;
    const uint64_t blocks = (waves * 64 + 255) / 256;
    hipLaunchKernelGGL(affine_generic_kernel, dim3(uint32_t(blocks)), dim3(256), 0, stream, a.w,
                       a.s, a.b, static_cast<int>(a.meta), a.x, a.y, a.rows, a.cols, a.bits,
                       a.group, a.batch);
    return hipGetLastError();
}

hipError_t launch_embed_affine(const uint32_t *w, const void *s, const void *b, Meta meta,
                               uint32_t row, uint32_t cols, uint32_t bits, uint32_t group,
                               float *y, hipStream_t stream) {
    hipLaunchKernelGGL(embed_affine_kernel, dim3((cols + 255) / 256), dim3(256), 0, stream, w, s,
                       b, static_cast<int>(meta), row, cols, bits, group, y);
    return hipGetLastError();
}

namespace {

// Rows per wave and waves per row group of the streaming dense kernel.
struct DenseShape {
    uint32_t r, ks;
};

// Eight rows per wave at four RHS (half the x loads per weight), else four.
// The four waves of a workgroup split K (four times the waves), except at
// three or more RHS where one wave per row group already gives four waves
// per SIMD on 256 CUs. Measured on MI355X (us, interleaved, one box), one
// wave per row group and four rows -> this rule:
//   5120x17408  B=1 36.6 -> 32.0, B=2 44.0 -> 38.0, B=3 50.4 -> 45.7, B=4 62.0 -> 44.4
//   17408x5120  B=1 33.1 -> 30.5, B=2 38.5 -> 38.2, B=3 43.7 (kept), B=4 47.3 -> 46.2
// Each case is the best of (4 or 8 rows) x (one or four waves per group).
DenseShape dense_shape(uint32_t rows, uint32_t batch) {
    const uint32_t r = batch == 4 ? 8u : 4u;
    const bool filled = rows / r >= 4u * 4u * 256u;
    return DenseShape{r, filled && batch >= 3 ? 1u : 4u};
}

template <int B, int R, int KS>
void launch_dense_stream(const uint16_t *w, const float *x, float *y, uint32_t rows, uint32_t cols,
                         uint32_t w_bytes, hipStream_t stream) {
    const uint32_t blocks = KS == 1 ? (rows + 4 * R - 1) / (4 * R) : (rows + R - 1) / R;
    hipLaunchKernelGGL((dense_f16_stream_kernel<B, R, KS>), dim3(blocks), dim3(256), 0, stream, w, x, y, rows,
                       cols, w_bytes);
}

template <int B>
void launch_dense_batch(DenseShape sh, const uint16_t *w, const float *x, float *y, uint32_t rows, uint32_t cols,
                        uint32_t w_bytes, hipStream_t stream) {
    if (sh.ks == 1) launch_dense_stream<B, 4, 1>(w, x, y, rows, cols, w_bytes, stream);
    else if (sh.r == 8) launch_dense_stream<B, 8, 4>(w, x, y, rows, cols, w_bytes, stream);
    else launch_dense_stream<B, 4, 4>(w, x, y, rows, cols, w_bytes, stream);
}

}  // namespace

hipError_t launch_dense_f16(const uint16_t *w, const float *x, float *y, uint32_t rows,
                            uint32_t cols, uint32_t batch, hipStream_t stream) {
    const uint64_t w_bytes = uint64_t(rows) * cols * 2;
    if (cols % 8 == 0 && w_bytes < (1ull << 31) && uint64_t(batch) * cols * 4 < (1ull << 31) && batch >= 1 &&
        batch <= 4) {
        const DenseShape sh = dense_shape(rows, batch);
        const uint32_t wb = uint32_t(w_bytes);
        switch (batch) {
            case 1: launch_dense_batch<1>(sh, w, x, y, rows, cols, wb, stream); break;
            case 2: launch_dense_batch<2>(sh, w, x, y, rows, cols, wb, stream); break;
            case 3: launch_dense_batch<3>(sh, w, x, y, rows, cols, wb, stream); break;
            default: launch_dense_batch<4>(sh, w, x, y, rows, cols, wb, stream); break;
        }
        return hipGetLastError();
    }
    const uint64_t waves = uint64_t(rows) * batch;
    const uint64_t blocks = (waves * 64 + 255) / 256;
    hipLaunchKernelGGL(dense_f16_kernel, dim3(uint32_t(blocks)), dim3(256), 0, stream, w, x, y,
                       rows, cols, batch);
    return hipGetLastError();
}

// The streaming kernel's time (us) as the read floor's fixed part plus the
// weight stream at the measured read rate, stretched per RHS count by the
// factor measured on MI355X over 2048x5120, 5120x5120, 5120x17408 and
// 17408x5120 (1.0-1.18 at one RHS, 1.34-1.48 at two, 1.64-1.84 at three,
// 1.67-2.36 at four; the middle of each range here).
double dense_valu_cost(uint32_t rows, uint32_t cols, uint32_t batch) {
    static constexpr double stretch[5] = {1.0, 1.1, 1.4, 1.72, 1.9};
    return 2.19 + double(rows) * cols * 2.0 / 6.98e6 * stretch[batch < 1 ? 1 : batch > 4 ? 4 : batch];
}

hipError_t launch_embed_f16(const uint16_t *w, uint32_t row, uint32_t cols, float *y,
                            hipStream_t stream) {
    hipLaunchKernelGGL(embed_f16_kernel, dim3((cols + 255) / 256), dim3(256), 0, stream, w, row,
                       cols, y);
    return hipGetLastError();
}

namespace {

typedef uint32_t copy_u4 __attribute__((ext_vector_type(4)));

// 16 bytes per lane per step, grid-stride; the scalar tail covers n % 4 and
// views that are not 16-byte aligned. An identical source and destination
// view (allowed by the dispatch contract) rewrites each element in place.
__global__ __launch_bounds__(256) void copy_f32_kernel(const float *__restrict__ x,
                                                       float *__restrict__ y, uint32_t n,
                                                       uint32_t vec) {
    const uint32_t stride = gridDim.x * blockDim.x;
    const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t nv = vec ? n / 4 : 0;
    const copy_u4 *xv = reinterpret_cast<const copy_u4 *>(x);
    copy_u4 *yv = reinterpret_cast<copy_u4 *>(y);
    for (uint32_t i = tid; i < nv; i += stride) __builtin_nontemporal_store(xv[i], yv + i);
    for (uint32_t i = nv * 4 + tid; i < n; i += stride) y[i] = x[i];
}

// Pure streaming read of three views (sizes in bytes, multiples of 4). The
// views' whole 16-byte chunks form one index space, cut into one contiguous
// slice per workgroup; each thread requests U chunks at once with 16-byte
// loads (non-temporal when NT; a view's chunk run may start at any 4-byte
// offset), so a workgroup's slice, which may span two views, costs one
// memory round trip per U chunks per thread. Slot g receives the XOR of
// workgroup g's words, the last workgroup also reads the views' trailing
// (bytes % 16) / 4 words, and workgroup 0 zeroes the slots past the grid.
template <int U, int NT>
__global__ __launch_bounds__(256) void read_checksum_kernel(const unsigned char *a, uint32_t na,
                                                            const unsigned char *b, uint32_t nb,
                                                            const unsigned char *c, uint32_t nc, uint32_t *out,
                                                            uint32_t slots) {
    const uint32_t G = gridDim.x, g = blockIdx.x, t = threadIdx.x;
    const uint32_t ca = na / 16, cab = ca + nb / 16, total = cab + nc / 16;
    const uint32_t per = (total + G - 1) / G;
    const uint32_t lo = g * per, hi = min(lo + per, total);
    uint32_t acc = 0;
    for (uint32_t k = lo + t; k < hi; k += 256u * U) {
        copy_u4 q[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t kk = k + 256u * u;
            const unsigned char *p = kk < ca ? a + size_t(kk) * 16u
                                   : kk < cab ? b + size_t(kk - ca) * 16u
                                              : c + size_t(kk - cab) * 16u;
            const copy_u4 *pv = reinterpret_cast<const copy_u4 *>(p);
            if constexpr (NT != 0) q[u] = kk < hi ? __builtin_nontemporal_load(pv) : copy_u4{0, 0, 0, 0};
            else q[u] = kk < hi ? *pv : copy_u4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= q[u][0] ^ q[u][1] ^ q[u][2] ^ q[u][3];
    }
    // Trailing words: lanes 0-2 of view a, 4-6 of b, 8-10 of c.
    if (g == G - 1 && t < 12 && (t & 3) < 3) {
        const uint32_t v = t >> 2, i = t & 3;
        const uint32_t n = v == 0 ? na : (v == 1 ? nb : nc);
        const unsigned char *base = v == 0 ? a : (v == 1 ? b : c);
        if (i < (n % 16) / 4) acc ^= *reinterpret_cast<const uint32_t *>(base + size_t(n / 16) * 16u + i * 4u);
    }
    __shared__ uint32_t red[4];
    for (int m = 32; m >= 1; m >>= 1) acc ^= uint32_t(__shfl_xor(int(acc), m, 64));
    if ((t & 63) == 0) red[t >> 6] = acc;
    __syncthreads();
    if (t == 0) out[g] = red[0] ^ red[1] ^ red[2] ^ red[3];
    if (g == 0)
        for (uint32_t i = G + t; i < slots; i += 256) out[i] = 0u;
}

}  // namespace

hipError_t launch_read_checksum(const void *a, uint32_t na, const void *b, uint32_t nb, const void *c, uint32_t nc,
                                uint32_t *out, const ReadPlan &plan, hipStream_t stream) {
    const uint64_t total = uint64_t(na) + nb + nc;
    // Default: about 48 KB per workgroup (four 16-byte non-temporal loads per
    // thread in flight), within [256, kChecksumSlots] workgroups. Measured on
    // MI355X over the metric matrix's 50.1 MB (back-to-back launches over 10
    // rotating copies): 1024 workgroups of 48 KB read it in 9.48-9.55 us,
    // against 9.71-9.83 us for 4080 workgroups of 12 KB (the previous
    // default), 11.6-11.8 us for 8160 and 15.3 us for 16320.
    uint64_t g = plan.workgroups ? plan.workgroups : (total + 49151) / 49152;
    if (!plan.workgroups && g < 256) g = 256;
    g = g < 1 ? 1 : (g > kChecksumSlots ? kChecksumSlots : g);
    const uint32_t u = plan.unroll ? plan.unroll : 4;
    const bool nt = plan.nt >= 0 ? plan.nt != 0 : true;
    auto *pa = static_cast<const unsigned char *>(a);
    auto *pb = static_cast<const unsigned char *>(b);
    auto *pc = static_cast<const unsigned char *>(c);
    const dim3 grid{uint32_t(g)}, block{256u};
    switch (u * 2 + (nt ? 1u : 0u)) {
        case 2: hipLaunchKernelGGL((read_checksum_kernel<1, 0>), grid, block, 0, stream, pa, na, pb, nb, pc, nc, out, kChecksumSlots); break;
        case 3: hipLaunchKernelGGL((read_checksum_kernel<1, 1>), grid, block, 0, stream, pa, na, pb, nb, pc, nc, out, kChecksumSlots); break;
        case 4: hipLaunchKernelGGL((read_checksum_kernel<2, 0>), grid, block, 0, stream, pa, na, pb, nb, pc, nc, out, kChecksumSlots); break;
        case 5: hipLaunchKernelGGL((read_checksum_kernel<2, 1>), grid, block, 0, stream, pa, na, pb, nb, pc, nc, out, kChecksumSlots); break;
        case 8: hipLaunchKernelGGL((read_checksum_kernel<4, 0>), grid, block, 0, stream, pa, na, pb, nb, pc, nc, out, kChecksumSlots); break;
        case 9: hipLaunchKernelGGL((read_checksum_kernel<4, 1>), grid, block, 0, stream, pa, na, pb, nb, pc, nc, out, kChecksumSlots); break;
        case 16: hipLaunchKernelGGL((read_checksum_kernel<8, 0>), grid, block, 0, stream, pa, na, pb, nb, pc, nc, out, kChecksumSlots); break;
        case 17: hipLaunchKernelGGL((read_checksum_kernel<8, 1>), grid, block, 0, stream, pa, na, pb, nb, pc, nc, out, kChecksumSlots); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Holds the stream for `ticks` of the constant-rate real-time counter: one
// wave polls the counter with long sleeps in between and always ends when
// the interval has passed. A benchmark enqueues it before its start mark so
// that every launch behind it is already queued when the GPU reaches them.
__global__ __launch_bounds__(64) void delay_kernel(unsigned long long ticks) {
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(127);
}

hipError_t launch_delay(unsigned long long ticks, hipStream_t stream) {
    hipLaunchKernelGGL(delay_kernel, dim3(1), dim3(64), 0, stream, ticks);
    return hipGetLastError();
}

// Zero fill with vector stores (a kernel rather than hipMemsetAsync, so that
// a command captured into a graph clears the memory on every replay).
__global__ __launch_bounds__(256) void zero_u32_kernel(uint32_t *__restrict__ p, uint32_t n) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0u;
}

hipError_t launch_zero_u32(uint32_t *p, uint32_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const uint32_t want = (n + 255) / 256;
    hipLaunchKernelGGL(zero_u32_kernel, dim3(want < 1024 ? want : 1024), dim3(256), 0, stream, p, n);
    return hipGetLastError();
}

hipError_t launch_copy_f32(const float *x, float *y, uint32_t n, int num_cus,
                           hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const bool vec = (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 16 == 0;
    const uint64_t items = vec ? (uint64_t(n) + 3) / 4 : n;
    const uint64_t want = (items + 255) / 256;
    const uint64_t cap = uint64_t(num_cus > 0 ? num_cus : 256) * 16;
    const uint32_t blocks = uint32_t(want < cap ? want : cap);
    hipLaunchKernelGGL(copy_f32_kernel, dim3(blocks), dim3(256), 0, stream, x, y, n,
                       uint32_t(vec));
    return hipGetLastError();
}

}  // namespace qmr

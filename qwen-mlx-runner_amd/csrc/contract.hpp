// Host-side dispatch contract: buffer-size layout, view checks, kernel
// selection and mode parsing. Pure C++ (no HIP) so it is testable on a CPU.
// Each function restates the reference's routine of the same name in
// src/gpu.rs (cited per function in contract.cpp).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

struct qmr_device;
struct qmr_buffer;

namespace qmr {

// Error carrying the reference's message text; converted to a status code and
// a thread-local message at the C-ABI boundary.
struct Error {
    int code;
    std::string message;
};

// The C-ABI's thread-local error message (qmr_last_error), for entry points
// defined outside runtime.cpp: record_error stores `message` and returns
// `code`; clear_error empties it at the start of a call.
int record_error(int code, const std::string &message);
void clear_error();

// Bytes of device memory currently free on the device's GPU (hipMemGetInfo);
// throws Error on a HIP failure.
size_t device_free_bytes(const ::qmr_device *device);

// Uploads from large pageable sources (mapped checkpoint shards) into new
// device buffers through pinned staging slots filled by several host
// threads, all views in one pipeline; returns QMR_OK or an error status with
// qmr_last_error() set (then no buffer is returned).
constexpr int kStageSlots = 3;
constexpr size_t kStageChunk = size_t(8) << 20;
struct StagedView {
    const void *src;
    size_t bytes;
};
int upload_staged_views(::qmr_device *device, const StagedView *views, size_t n, ::qmr_buffer **outs);
int upload_staged(::qmr_device *device, const void *src, size_t bytes, ::qmr_buffer **out);

enum class BlockMatmulMode : int { Legacy = 0, Shared = 1, MlpR2 = 2 };

struct BlockKernelMode {
    BlockMatmulMode matmul = BlockMatmulMode::Legacy;
    bool batched_delta = true;
};

struct Layout {
    std::vector<size_t> sizes;  // minimum byte size of each buffer view
    size_t threads = 0;         // logical thread count of the reference ABI
};

// Metadata storage of a packed matrix on the device.
enum class Meta : int { F32 = 0, BF16 = 1, F16 = 2 };

// Throws Error on any violation, with the reference's message.
Layout dispatch_layout(const std::string &name, const uint32_t *p, size_t n);
void checked_buffer_range(size_t offset, size_t minimum, size_t length);
bool ranges_overlap(size_t a, size_t a_len, size_t b, size_t b_len);

const char *specialized_matvec(const uint32_t *p, bool aligned);
const char *specialized_matvec_bf16(const uint32_t *p, bool aligned);
const char *specialized_matmul(const std::string &name, const uint32_t *p, bool aligned,
                               BlockMatmulMode mode);

BlockKernelMode parse_block_kernel_mode(const char *matmul, const char *delta);
BlockKernelMode parse_block_kernel_mode_for_device(const std::string &device_name,
                                                   const char *matmul, const char *delta);

bool supported_bf16_quantization(uint32_t bits, size_t group);
bool pack_bf16_exact(const float *values, size_t n, uint16_t *out);

// Name helpers.
bool starts_with(const std::string &s, const char *prefix);
bool ends_with(const std::string &s, const char *suffix);
// Metadata storage implied by a reference (or added) kernel name.
Meta meta_of_name(const std::string &name);
bool is_affine_matrix_name(const std::string &name);  // matvec/matmul affine family
bool is_block_name(const std::string &name);          // matmul_affine*, matmul_f16
bool is_wide_name(const std::string &name);           // matmul_affine_wide*
// Fused names with no reference counterpart: matmul_affine_add[_bf16|_f16meta]
// (y = r + W x) and mlp_gate_up_swiglu[_bf16|_f16meta] (RMS norm, gate and up
// products and SwiGLU in one launch).
bool is_residual_name(const std::string &name);
bool is_mlp_name(const std::string &name);
bool is_fused_name(const std::string &name);
// read_checksum: u32 checksum slots written per launch (the XOR of all of
// them is the XOR of every 32-bit word read).
constexpr uint32_t kChecksumSlots = 4096;

}  // namespace qmr

/*
 * qmr.h -- C ABI of the MI355X (gfx950) backend for qwen-mlx-runner's matrix
 * dispatch surface: fused dequantisation + GEMV / small-block / wide-block
 * products over MLX affine packed Q4/Q8 weights (uint32-packed codes,
 * per-group scale and bias, w = scale*q + bias).
 *
 * The surface mirrors the reference engine's Metal backend (`Gpu` and
 * `DispatchEncoder` in src/gpu.rs), which every caller of the hot path goes
 * through: `Matrix::{matvec,embed}` (src/engine.rs:137-188) and
 * `Matrix::{matmul_block,embed_offset}` (src/engine/block.rs:191-261).
 * Kernel names, parameter words, buffer order, byte-offset views, the
 * host-side validation contract and the kernel-selection predicates are the
 * reference's; the kernels behind them are this library's own HIP code.
 *
 * Conventions
 *   - Every call that can fail returns QMR_OK (0) or a nonzero status and
 *     leaves a message in a thread-local slot read by qmr_last_error().
 *   - Validation happens before any side effect: a rejected qmr_encode
 *     enqueues nothing (src/gpu.rs:638-792).
 *   - A device handle is used by one thread at a time (the reference's `Gpu`
 *     is !Sync, src/gpu.rs:105-109). All work of one command is enqueued on
 *     the device's single HIP stream and synchronised once by
 *     qmr_command_finish, like one Metal command buffer per token.
 *   - GPU execution failures surface at qmr_command_finish (src/gpu.rs:861-865).
 *   - Plain pointers and sizes only; no C++ or framework types.
 */
#ifndef QMR_H
#define QMR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QMR_OK 0
#define QMR_ERR_INVALID 1     /* argument / shape / view validation failed */
#define QMR_ERR_DEVICE 2      /* HIP runtime or device failure */
#define QMR_ERR_UNSUPPORTED 3 /* no kernel for this specialisation */

/* Block-matmul schedules (src/gpu.rs:22-31, BlockMatmulMode). */
#define QMR_BLOCK_LEGACY 0
#define QMR_BLOCK_SHARED 1
#define QMR_BLOCK_MLP_R2 2

typedef struct qmr_device qmr_device;
typedef struct qmr_buffer qmr_buffer;
typedef struct qmr_command qmr_command;

/* Device options. Each replaces an environment variable the reference reads
 * in Gpu::new* (src/gpu.rs:294-325, 49-92); NULL selects the reference's
 * default. Strings are validated with the reference's exact accepted sets. */
typedef struct {
    const char *gemv_variant;  /* QWEN_METAL_GEMV: "aligned" (default) | "packed4" | "stream" */
    const char *metadata_mode; /* QWEN_METAL_METADATA: "f32" (default) | "bf16" */
    const char *block_matmul;  /* QWEN_METAL_BLOCK_MATMUL: "legacy" | "shared" | "mlp-r2";
                                  NULL = device default (src/gpu.rs:49-60) */
    const char *block_delta;   /* QWEN_METAL_BLOCK_DELTA: "sequential" | "batched" (default) */
    int reference;             /* QWEN_METAL_REFERENCE=1: reference arithmetic mode */
} qmr_device_options;

/* Replaces FrameTiming (src/gpu/timing.rs:8-21). gpu_seconds is device time:
 * from a HIP event recorded on the device stream right before the command's
 * first launch (after any workspace growth) to one recorded at finish, so
 * host time before the first encode is not counted (a command that launched
 * nothing reports about zero). */
typedef struct {
    double cpu_encode_seconds;
    double cpu_commit_seconds;
    double gpu_seconds;
    double completion_wait_seconds;
} qmr_frame_timing;

/* Message of the last failed call on this thread ("" if none). */
const char *qmr_last_error(void);

/* ---- Device: replaces Gpu::new_with_variant (src/gpu.rs:305-437) ---- */
int qmr_device_open(int ordinal, const qmr_device_options *options, qmr_device **out);
void qmr_device_close(qmr_device *device);
/* HIP device name (gcnArchName-qualified marketing name). */
const char *qmr_device_name(const qmr_device *device);
/* Gpu::kernel_mode (src/gpu.rs:438-444): "reference" or the GEMV variant. */
const char *qmr_kernel_mode(const qmr_device *device);
/* Gpu::metadata_mode (src/gpu.rs:467-471). */
const char *qmr_metadata_mode(const qmr_device *device);
/* Gpu::block_kernel_mode / set_block_kernel_mode (src/gpu.rs:445-452). Call
 * only between completed commands. */
void qmr_block_kernel_mode(const qmr_device *device, int *matmul, int *batched_delta);
int qmr_set_block_kernel_mode(qmr_device *device, int matmul, int batched_delta);
/* Gpu::compact_metadata (src/gpu.rs:479-490): returns 1 and fills s_out/b_out
 * (n u16 each) when BF16 metadata is enabled, the format is supported and
 * both arrays compact losslessly; 0 otherwise (caller keeps FP32). */
int qmr_compact_metadata(const qmr_device *device, uint32_t bits, size_t group,
                         const float *scales, const float *biases, size_t n,
                         uint16_t *s_out, uint16_t *b_out);
/* Gpu::record_compacted_metadata / metadata_stats (src/gpu.rs:472-478,491-496). */
void qmr_record_compacted_metadata(qmr_device *device, uint64_t saved_bytes);
void qmr_metadata_stats(const qmr_device *device, size_t *matrices, uint64_t *saved_bytes);

/* ---- Buffers: replace Gpu::{alloc_f32,upload_bytes,upload_f32,read_f32}
 * (src/gpu.rs:540-589) and Metal's refcounted buffer handles
 * (Matrix::share, src/engine.rs:35-46). A new handle holds one reference. */
/* Zero-filled allocation of max(bytes, 4) bytes (alloc_f32 semantics). */
int qmr_buffer_alloc(qmr_device *device, size_t bytes, qmr_buffer **out);
/* Copy host bytes into a new device buffer; empty input yields a 4-byte
 * zero buffer, as upload_bytes does. */
int qmr_buffer_upload(qmr_device *device, const void *data, size_t bytes, qmr_buffer **out);
/* Copy bytes [offset, offset+bytes) to the host. Valid only after the
 * command that last wrote the buffer has finished (src/gpu.rs:577). */
int qmr_buffer_read(const qmr_buffer *buffer, size_t offset, void *dst, size_t bytes);
/* Overwrite bytes of an existing buffer from the host (synchronous). */
int qmr_buffer_write(qmr_buffer *buffer, size_t offset, const void *src, size_t bytes);
size_t qmr_buffer_length(const qmr_buffer *buffer);
void qmr_buffer_retain(qmr_buffer *buffer);
void qmr_buffer_release(qmr_buffer *buffer);

/* ---- Commands: replace Gpu::begin / DispatchEncoder / Gpu::finish
 * (src/gpu.rs:590-876). ---- */
int qmr_command_begin(qmr_device *device, qmr_command **out);
/* DispatchEncoder::encode / encode_offsets (src/gpu.rs:120-141):
 * `name` is a reference kernel name (matvec_affine, matvec_affine_bf16,
 * matmul_affine, matmul_affine_bf16, embed_affine, embed_affine_bf16,
 * matvec_f16, matmul_f16, embed_f16, copy_f32) or one of this library's additions
 * (matmul_affine_wide[_bf16], see below). `offsets` may be NULL (all zero) or
 * hold one 4-byte-aligned byte offset per buffer. `params`, `threads` and
 * `group_size` follow dispatch_layout (src/gpu.rs:1041-1294). */
int qmr_encode(qmr_command *command, const char *name, qmr_buffer *const *buffers,
               const size_t *offsets, size_t nbuffers, const uint32_t *params,
               size_t nparams, size_t threads, size_t group_size);
/* No counterpart in the reference: qmr_encode for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc). Same arguments, validation and kernels;
 * it calls no hipMalloc, hipFree or allocating library routine. The
 * workspace its kernels need (the row-band kernel's split sums, the split-K
 * kernel's partial sums and counters, the wide block's activation images)
 * comes from a static scratch array of QMR_STATIC_SCRATCH_BYTES that each GPU
 * holds from library load until the process ends; a launch needing more is
 * rejected with QMR_ERR_INVALID before anything is enqueued. Workspace that
 * must start at zero (split sums tagged with a fixed epoch, arrival counters)
 * is cleared by a fill kernel inside the call when earlier launches may have
 * left it non-zero: the split-K kernel and the row-band kernel's GEMV and
 * block forms (plain or residual) clear every slot and counter they take, so
 * after the first fill the region stays zero from call to call and needs no
 * fill until the wide block, the row-band MLP form or a failed command has
 * used it. All calls on one GPU share its scratch: calls whose launches
 * overlap in time (other streams, other device handles on the same GPU)
 * race. */
#define QMR_STATIC_SCRATCH_BYTES (8u << 20)
int qmr_encode_static(qmr_command *command, const char *name, qmr_buffer *const *buffers,
                      const size_t *offsets, size_t nbuffers, const uint32_t *params,
                      size_t nparams, size_t threads, size_t group_size);
/* Records a HIP event on the device stream; *index identifies it for
 * qmr_command_elapsed after the command finishes. (The Metal backend's
 * counterpart is the GPU start/end timestamp pair of FrameTiming.) */
int qmr_command_mark(qmr_command *command, int *index);
/* No counterpart in the reference (a measurement aid): enqueues one wave
 * that holds the device stream for `microseconds` (at most 1,000,000) of
 * the GPU's real-time clock. A benchmark calls it before its start mark so
 * that the launches it enqueues next are all queued when the GPU reaches
 * them, and the marks time them back to back whatever the host's enqueue
 * rate. */
int qmr_command_delay(qmr_command *command, uint32_t microseconds);
/* Gpu::finish: synchronise, check status, fill timing (may be NULL). */
int qmr_command_finish(qmr_command *command, qmr_frame_timing *timing);
/* Milliseconds between two marks of a finished command. */
int qmr_command_elapsed(const qmr_command *command, int from, int to, double *ms);
void qmr_command_release(qmr_command *command);

/* ---- Host-only contract functions (no device needed). These restate the
 * reference's validation and routing so that they can be tested on a CPU,
 * as the reference tests them (src/gpu.rs:1295-1634). ---- */
/* dispatch_layout (src/gpu.rs:1041-1294), matrix kernels: required byte size
 * of each buffer view and the logical thread count. */
int qmr_dispatch_layout(const char *name, const uint32_t *params, size_t nparams,
                        size_t *sizes, size_t max_sizes, size_t *nsizes, size_t *threads);
/* checked_buffer_range / ranges_overlap (src/gpu.rs:879-894). */
int qmr_checked_buffer_range(size_t offset, size_t minimum, size_t length);
int qmr_ranges_overlap(size_t a, size_t a_len, size_t b, size_t b_len);
/* specialized_matvec / specialized_matvec_bf16 (src/gpu.rs:1003-1037);
 * returns the reference pipeline name or NULL. */
const char *qmr_specialized_matvec(const uint32_t *params, int aligned, int bf16);
/* specialized_matmul (src/gpu.rs:896-999). */
const char *qmr_specialized_matmul(const char *name, const uint32_t *params, size_t nparams,
                                   int aligned, int mode);
/* BlockKernelMode::parse_for_device (src/gpu.rs:49-77); NULL = unset. */
int qmr_parse_block_kernel_mode(const char *device_name, const char *matmul, const char *delta,
                                int *matmul_out, int *batched_delta_out);
/* pack_bf16_exact / supported_bf16_quantization (src/gpu/metadata.rs:6-18). */
int qmr_pack_bf16_exact(const float *values, size_t n, uint16_t *out);
int qmr_supported_bf16_quantization(uint32_t bits, size_t group);

/*
 * Kernel names with no counterpart in the reference:
 *   "matmul_affine_wide" / "matmul_affine_wide_bf16"
 *     The reference caps blocks at four RHS (src/gpu.rs:1136-1140). Buffers
 *     w, s, b, x, y; params rows, cols, bits, group, batch with
 *     1 <= batch <= 256; x [batch][cols], y [batch][rows] token-major;
 *     threads = rows*32. Q4/g64 runs on MFMA; meant for chunked prefill.
 *     Batches of up to eight run as successive blocks of up to four.
 *   "matmul_affine_add" / "_bf16" / "_f16meta"
 *     y = r + W x, the down projection with the decoder's residual add
 *     (src/engine.rs:764-765). Buffers w, s, b, x, r, y; params as the
 *     blocks (batch 1..4); r and y [batch][rows]; y may be exactly r's view
 *     (in place), any other overlap is rejected. Matrix-core formats only.
 *   "mlp_gate_up_swiglu" / "_bf16" / "_f16meta"
 *     y = silu(G n) * (U n), n = rms_norm(x, norm, eps): the decoder MLP's
 *     rms_norm + gate + up + swiglu (src/engine.rs:748-763) in one launch.
 *     Buffers gate w/s/b, up w/s/b (same shape and format), x [batch][cols],
 *     norm [cols], y [batch][rows]; params rows, cols, bits, group, batch
 *     (1..4), eps as FP32 bits (finite, positive). Matrix-core formats only.
 *   "read_checksum"
 *     One streaming read of three byte views: buffers a, b, c, out; params
 *     the three sizes in bytes (multiples of 4, not all zero); threads =
 *     ceil((a+b+c)/16). out holds 4096 u32 slots whose XOR is the XOR of
 *     every 32-bit word read. The read floor of a product's codes and
 *     metadata, for measurement; it computes nothing else.
 *   "matvec_affine_f16meta", "matmul_affine_f16meta", "embed_affine_f16meta"
 *     As the FP32-metadata names, with scales/biases stored as IEEE binary16
 *     (the dtype MLX checkpoints ship). The reference expands F16 metadata
 *     to FP32 on load (src/weights.rs:436-437); storing it as 16 bits cuts
 *     metadata bytes in half. Same layout rules as the _bf16 names.
 */

/* ---- Testing and tuning hooks (no counterpart in the reference). ---- */
/* Force the GEMV kernel and tiling; 0,0 = planner (the row-band matrix-core
 * kernel where it has a one-round plan, or, for matrices too tall for one
 * round, single-split bands over several rounds; else the split-K
 * matrix-core kernel where supported, the row-owning one past one round of
 * resident workgroups or for splits under four K tiles, else the vector-ALU
 * kernels). The fused MLP form: the row-band kernel's MLP form where it has
 * a one-round plan, else split-K's, else the row-owning kernel's.
 *   rr = -3: row-owning matrix-core kernel (also its MLP form); ks =
 *            j*10000 + rt*100 + kw pins its workgroup shape (rt row tiles x
 *            kw K waves) and, when j > 0, the entries per wave per staged
 *            chunk; 0 = its planner.
 *   rr = -2: split-K matrix-core kernel; ks > 0 keeps only that number of
 *            K splits when it is feasible (else the planner's count), 0 =
 *            its planner.
 *   rr = -1: the vector-ALU streaming single-RHS kernel (blocks then use
 *            the row-slot tiling).
 *   rr > 0 with ks > 0: the vector-ALU row-slot kernel with `rr` rows per
 *            slot and a K-split of `ks`.
 *   rr = -4: row-band matrix-core kernel; ks = phases*1000000 +
 *            ring*100000 + ns*10000 + tr*100 + kw pins its x staging
 *            phases (1, or 2 for single-split plans of one wave per tile),
 *            ring depth (2 or 3), K splits (1-8; its planner takes at most
 *            4), row tiles per band (the MLP form: tr/2 gate and tr/2 up
 *            tiles) and waves per tile; zero fields and ks = 0 leave them
 *            to its planner.
 *   rr = -5: dense F16 products (matvec_f16, matmul_f16) on the matrix-core
 *            kernel with ks = ring*10000 + kw*1000 + rt*100 + ns (entries
 *            in flight per wave, 4 or 8; waves per row tile; row tiles per
 *            workgroup; K splits; zero fields and ks = 0 leave them to its
 *            planner). Dense
 *            products run on that kernel by default wherever it supports
 *            the view (16-byte aligned weights, cols % 32 == 0); rr = -1
 *            sends them to the vector-ALU kernels.
 * Shapes a forced kernel does not support fall back to the next one; pairs
 * that are not compiled fall back to the planner. */
int qmr_set_gemv_plan(qmr_device *device, int rr, int ks);
/* The plan the GEMV launcher uses for a shape with group 64 and BF16
 * metadata (honours a forced plan), in the encoding of qmr_set_gemv_plan;
 * the row-band kernel reports rr = -4 with its ks (phases 2 as
 * 2000000 + ..., one phase without the digit), the split-K kernel
 * rr = -2 with ks = its K splits. bits = 16: the plan of a dense F16
 * product over an aligned view (rr = -5 with its ks, or rr = -1 for the
 * vector-ALU kernels). */
int qmr_gemv_plan(const qmr_device *device, uint32_t rows, uint32_t cols, uint32_t bits,
                  uint32_t batch, int *rr, int *ks);
/* Tuning hook for "read_checksum" (the read floor a product is measured
 * against): workgroups of 256 threads (1..4096; 0 = about 48 KB each),
 * 16-byte loads each thread keeps in flight (1, 2, 4 or 8; 0 = 4), and
 * non-temporal (1) or plain (0) loads (-1 = the default, non-temporal). */
int qmr_set_read_plan(qmr_device *device, uint32_t workgroups, uint32_t unroll, int nontemporal);
/* Testing hook for the failure path of qmr_command_finish: while enabled,
 * the last K splits of the row-band and split-K kernels wait for sums that no
 * split of the launch publishes and give up after a short bound (every
 * workgroup still exits), as the row-band kernel's would if a band's
 * workgroups were not all resident at once; the command's finish then
 * returns QMR_ERR_DEVICE naming the kernel and band. */
int qmr_set_band_wait_fault(qmr_device *device, int enabled);
/* Bytes of device workspace this handle has allocated for its kernels (the
 * row-band split sums, the split-K partial sums and counters, the wide
 * block's activation images); qmr_encode_static allocates none. */
size_t qmr_device_workspace_bytes(const qmr_device *device);
/* Reference pipeline label selected by the last successful qmr_encode. */
const char *qmr_last_kernel(const qmr_device *device);
/* The HIP kernel the last qmr_encode launched (with the row-band kernel's
 * plan: "affine_band_kernel ring=R ns=S tr=T kw=K"), or the encode name for
 * families with a single kernel. */
const char *qmr_last_hip_kernel(const qmr_device *device);
/* LDS bytes one workgroup may allocate on this device. */
size_t qmr_device_max_lds(const qmr_device *device);
/* Host-only check of the wide block kernel's addressing (no device needed):
 * walks every code, x-fragment and group-sum load its contraction launch
 * issues for rows x cols (a multiple of 256) times batch RHS with row_tiles
 * (8 or 17) 16-row tiles per workgroup, and writes out[0] = the largest end
 * (byte offset + size) of the in-range code loads, out[1] = the code view's
 * size, out[2] = the largest end of the in-range image loads, out[3] = the
 * image workspace's size. Loads outside a view take the vector offset past
 * every view and read zeros. */
int qmr_wide_address_extent(uint32_t rows, uint32_t cols, uint32_t batch, uint32_t row_tiles, uint64_t *out);

#ifdef __cplusplus
}
#endif
#endif /* QMR_H */

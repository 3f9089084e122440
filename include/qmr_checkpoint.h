/* MLX checkpoint loader: safetensors shards with MLX affine quantisation
 * metadata, read into host arrays or straight into device buffers.
 *
 * Replaces the reference's `Checkpoint` (src/weights.rs:32-73,168-486,569-738)
 * and `Matrix::load` (src/engine.rs:48-135) for the matrices the packed-affine
 * products consume. Model-level parts of the reference's checkpoint (the model
 * configuration, norm sanitising, convolution layouts, vectors, MTP adapters)
 * are not on this path and are not provided.
 *
 * Conventions are those of qmr.h: every call that can fail returns QMR_OK or
 * a nonzero status and leaves a message in qmr_last_error(). A checkpoint
 * handle is immutable after qmr_checkpoint_open and may be read from several
 * threads; it keeps its shards memory-mapped until qmr_checkpoint_close.
 */
#ifndef QMR_CHECKPOINT_H
#define QMR_CHECKPOINT_H

#include <stddef.h>
#include <stdint.h>

#include "qmr.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qmr_checkpoint qmr_checkpoint;

/* Checkpoint::open + from_config (src/weights.rs:56-73,168-290): reads
 * config.json (its "quantization" or else "quantization_config" object and
 * "tie_word_embeddings"), then either model.safetensors.index.json and every
 * shard it names, or the directory's single *.safetensors file. Each shard is
 * validated as parse_safetensors does (src/weights.rs:569-677): header length
 * at most 100 MB, strict JSON without duplicate keys, string-only
 * __metadata__, known dtypes, non-zero dimensions, byte lengths that match
 * shape x dtype, data ranges that tile the data section exactly. Tensor names
 * are canonicalised (canonical_name, src/weights.rs:458-472). */
int qmr_checkpoint_open(const char *dir, qmr_checkpoint **out);
void qmr_checkpoint_close(qmr_checkpoint *checkpoint);

/* Number of tensors across all shards. */
size_t qmr_checkpoint_tensor_count(const qmr_checkpoint *checkpoint);

/* Checkpoint::contains (src/weights.rs:389-395): 1 if the matrix or tensor
 * exists (a tied lm_head counts as present when the embedding is), else 0. */
int qmr_checkpoint_contains(const qmr_checkpoint *checkpoint, const char *name);

typedef struct qmr_matrix_info {
    int packed;              /* 1: U32 codes with scales and biases; 0: dense */
    size_t rows;
    size_t cols;             /* logical columns; packed: groups * group_size */
    uint32_t bits;           /* 4 or 8 when packed, 16 when dense */
    size_t group_size;       /* 0 when dense */
    char dtype[8];           /* stored dtype of the weight tensor */
    char metadata_dtype[8];  /* stored dtype of scales and biases ("" if dense) */
} qmr_matrix_info;

/* The shape and format Checkpoint::matrix (src/weights.rs:292-351) would
 * return for `name` ("model.layers.0.mlp.gate_proj" or with ".weight"),
 * with all of its checks: quantisation spec from the per-module override or
 * the default, bits 4 or 8, group a multiple of the codes per word, packed
 * width divisible by the words per group, scales/biases of shape
 * [rows, groups]. */
int qmr_checkpoint_matrix_info(const qmr_checkpoint *checkpoint, const char *name,
                               qmr_matrix_info *info);

/* Checkpoint::matrix, packed case (src/weights.rs:299-337): copies the
 * words (little-endian U32, rows * cols / (32 / bits) of them) and the
 * scales and biases expanded exactly to FP32 (rows * cols / group_size each;
 * non-finite metadata is rejected, src/weights.rs:416-445). */
int qmr_checkpoint_matrix(const qmr_checkpoint *checkpoint, const char *name, uint32_t *weights,
                          float *scales, float *biases);

/* Checkpoint::matrix, dense case (src/weights.rs:338-350): rows * cols F16
 * bit patterns, each value converted with round-to-nearest-even; values that
 * are non-finite or beyond +-65504 are rejected. */
int qmr_checkpoint_dense(const qmr_checkpoint *checkpoint, const char *name, uint16_t *values);

/* A matrix resident on one device (the reference's `Matrix`,
 * src/engine.rs:22-31). Dense matrices have no scales or biases, bits 16 and
 * group 0. */
typedef struct qmr_matrix {
    qmr_buffer *weight;
    qmr_buffer *scales;
    qmr_buffer *biases;
    size_t rows;
    size_t cols;
    uint32_t bits;
    size_t group;
    int metadata_bf16; /* scales and biases stored as BF16 bit patterns */
} qmr_matrix;

/* Matrix::load (src/engine.rs:48-135): reads `name`, checks that it is
 * [rows, cols], and uploads the codes unchanged (straight from the mapped
 * shard) and the metadata as FP32, or as BF16 when the device's metadata
 * mode is "bf16" and both arrays compact losslessly (qmr_compact_metadata;
 * recorded with qmr_record_compacted_metadata). Fails before allocating if
 * the upload would not fit in the device's free memory. On failure no
 * buffer is left allocated. */
int qmr_matrix_load(qmr_device *device, const qmr_checkpoint *checkpoint, const char *name,
                    size_t rows, size_t cols, qmr_matrix *out);

/* Releases the matrix's buffers (the reference drops its `Matrix`). */
void qmr_matrix_release(qmr_matrix *matrix);

#ifdef __cplusplus
}
#endif

#endif /* QMR_CHECKPOINT_H */

/*
 * qmr_oracle.c -- CPU oracle for the packed-affine GEMV / small-block hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or
 * calls this file. Its only users are tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, and there only as the checker (or as the CPU
 * path timed beside the GPU), never as the thing measured on the GPU.
 *
 * It restates, statement for statement, the FP64 closures the reference uses
 * to check its Metal kernels (paths relative to the reference repository):
 *   - tests/quantized.rs:39-51      per-weight unpack, affine, FP64 accumulate
 *   - tests/bf16_metadata.rs:41-56  BF16 metadata expanded as (u16 << 16)
 *   - tests/batch_matrix.rs:35-49   token-major blocks X[b*cols+c], Y[b*rows+r]
 *   - kernels/qwen.metal:40-47      affine(): q = (word >> ((c%pack)*bits)) & mask,
 *                                   gi = row*(cols/group) + col/group
 *   - kernels/affine_bf16.metal:162-174 / kernels/qwen.metal:73-77 embedding
 *                                   (row dequantisation, y[c] = q*s + b)
 *   - src/weights.rs:427-444        F16 / BF16 / F32 metadata decoding
 *   - src/gpu/metadata.rs:6-18      lossless FP32 -> BF16 metadata compaction
 *
 * Each exported function below names the line range it follows. Pinning (how
 * each function is checked against the reference's own known answers, its
 * fixture bytes and closed forms) lives in tests/test_oracle.py.
 *
 * Metadata kinds: 0 = FP32 values, 1 = BF16 bit patterns (u16), 2 = F16 bit
 * patterns (u16, IEEE binary16; the reference's `half` 2.7.1 decoding).
 */
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

enum { ORACLE_META_F32 = 0, ORACLE_META_BF16 = 1, ORACLE_META_F16 = 2 };

/* BF16 -> FP32: the stored u16 is the high half of the FP32 bit pattern.
 * Follows kernels/affine_bf16.metal:17-19 and tests/bf16_metadata.rs:53-56. */
float oracle_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* IEEE binary16 -> FP32, exact for every pattern (normals, subnormals, signed
 * zero, infinities, NaN payload kept quiet). Written from the IEEE-754 format
 * definition; it is what src/weights.rs:436-437 obtains from `half` 2.7.1. */
float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* Subnormal: value = man * 2^-24; normalise into FP32. */
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while ((man & 0x400) == 0);
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13) | (man ? 0x00400000u : 0);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Metadata element i as FP32, per src/weights.rs:430-441 (F32/F16/BF16). */
float oracle_meta(const void *meta, size_t i, int kind) {
    if (kind == ORACLE_META_F32) return ((const float *)meta)[i];
    uint16_t h = ((const uint16_t *)meta)[i];
    return kind == ORACLE_META_BF16 ? oracle_bf16_to_f32(h) : oracle_f16_to_f32(h);
}

/* Packed code at (row, col): kernels/qwen.metal:40-44 and tests/quantized.rs:41-44. */
uint32_t oracle_code(const uint32_t *w, size_t cols, uint32_t bits, size_t row, size_t col) {
    size_t pack = 32 / bits;
    uint32_t word = w[row * (cols / pack) + col / pack];
    return (word >> ((col % pack) * bits)) & ((1u << bits) - 1u);
}

/* Row dequantisation (the embedding kernels, kernels/qwen.metal:73-77 and
 * kernels/affine_bf16.metal:162-174): y[c] = float(q)*s + b, the product and
 * the sum each rounded to FP32. (With BF16 or F16 metadata the product is
 * exact, so this is also RN32(q*s + b).) */
void oracle_dequant_row(const uint32_t *w, const void *s, const void *b, int kind,
                        size_t row, size_t cols, uint32_t bits, size_t group, float *out) {
    for (size_t c = 0; c < cols; ++c) {
        uint32_t q = oracle_code(w, cols, bits, row, c);
        size_t gi = row * (cols / group) + c / group;
        /* float(q) * s + b with each operation rounded (kernels/qwen.metal:40-47,
         * 73-77); the Makefile builds with -ffp-contract=off. */
        const float prod = (float)q * oracle_meta(s, gi, kind);
        out[c] = prod + oracle_meta(b, gi, kind);
    }
}

/* FP64 oracle over a row range: tests/quantized.rs:39-51 generalised to the
 * token-major block of tests/batch_matrix.rs:35-49.
 *   y[t*rows + r] = sum_c (q * (f64)s + (f64)b) * (f64)x[t*cols + c]
 * summed in column order c = 0..cols-1, exactly as the reference's iterator. */
static void matmul_f64_rows(const uint32_t *w, const void *s, const void *b, int kind,
                            const float *x, double *y, size_t rows, size_t cols,
                            uint32_t bits, size_t group, size_t batch,
                            size_t row_begin, size_t row_end) {
    for (size_t t = 0; t < batch; ++t) {
        const float *xt = x + t * cols;
        for (size_t r = row_begin; r < row_end; ++r) {
            double acc = 0.0;
            for (size_t c = 0; c < cols; ++c) {
                uint32_t q = oracle_code(w, cols, bits, r, c);
                size_t gi = r * (cols / group) + c / group;
                acc += ((double)q * (double)oracle_meta(s, gi, kind) +
                        (double)oracle_meta(b, gi, kind)) * (double)xt[c];
            }
            y[t * rows + r] = acc;
        }
    }
}

/* FP32-accumulating variant of the same per-weight dequantise-then-multiply
 * loop, used only as a second (faster, fairer) CPU timing baseline. */
static void matmul_f32_rows(const uint32_t *w, const void *s, const void *b, int kind,
                            const float *x, float *y, size_t rows, size_t cols,
                            uint32_t bits, size_t group, size_t batch,
                            size_t row_begin, size_t row_end) {
    size_t pack = 32 / bits;
    uint32_t mask = (1u << bits) - 1u;
    size_t groups = cols / group;
    for (size_t t = 0; t < batch; ++t) {
        const float *xt = x + t * cols;
        for (size_t r = row_begin; r < row_end; ++r) {
            const uint32_t *wr = w + r * (cols / pack);
            float acc = 0.0f;
            for (size_t g = 0; g < groups; ++g) {
                float sv = oracle_meta(s, r * groups + g, kind);
                float bv = oracle_meta(b, r * groups + g, kind);
                for (size_t c = g * group; c < (g + 1) * group; ++c) {
                    uint32_t q = (wr[c / pack] >> ((c % pack) * bits)) & mask;
                    acc += ((float)q * sv + bv) * xt[c];
                }
            }
            y[t * rows + r] = acc;
        }
    }
}

typedef struct {
    const uint32_t *w;
    const void *s, *b;
    int kind;
    const float *x;
    void *y;
    size_t rows, cols, group, batch, row_begin, row_end;
    uint32_t bits;
    int f64;
} oracle_job;

static void *oracle_worker(void *arg) {
    oracle_job *j = (oracle_job *)arg;
    if (j->f64)
        matmul_f64_rows(j->w, j->s, j->b, j->kind, j->x, (double *)j->y, j->rows, j->cols,
                        j->bits, j->group, j->batch, j->row_begin, j->row_end);
    else
        matmul_f32_rows(j->w, j->s, j->b, j->kind, j->x, (float *)j->y, j->rows, j->cols,
                        j->bits, j->group, j->batch, j->row_begin, j->row_end);
    return NULL;
}

/* Validates the same shape contract as the reference's dispatch_layout
 * (src/gpu.rs:1097-1110): bits 4 or 8, cols divisible by the pack width and
 * by the group. Returns 0 on success, -1 on an invalid shape. */
static int oracle_shape_ok(size_t rows, size_t cols, uint32_t bits, size_t group, size_t batch) {
    if (!(bits == 4 || bits == 8) || group == 0 || rows == 0 || cols == 0 || batch == 0) return -1;
    if (cols % (32 / bits) != 0 || cols % group != 0) return -1;
    return 0;
}

static int oracle_run(const uint32_t *w, const void *s, const void *b, int kind,
                      const float *x, void *y, size_t rows, size_t cols, uint32_t bits,
                      size_t group, size_t batch, int threads, int f64) {
    if (oracle_shape_ok(rows, cols, bits, group, batch) != 0) return -1;
    if (threads < 1) threads = 1;
    if ((size_t)threads > rows) threads = (int)rows;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    oracle_job jobs[256];
    for (int i = 0; i < threads; ++i) {
        oracle_job j = {w, s, b, kind, x, y, rows, cols, group, batch,
                        rows * (size_t)i / (size_t)threads,
                        rows * (size_t)(i + 1) / (size_t)threads, bits, f64};
        jobs[i] = j;
    }
    int started = 0;
    for (int i = 1; i < threads; ++i) {
        if (pthread_create(&tid[i], NULL, oracle_worker, &jobs[i]) != 0) break;
        started = i;
    }
    oracle_worker(&jobs[0]);
    for (int i = 1; i <= started; ++i) pthread_join(tid[i], NULL);
    for (int i = started + 1; i < threads; ++i) oracle_worker(&jobs[i]);
    return 0;
}

/* y: double[batch*rows], token-major. Threads split rows; every output is
 * still summed by one thread in column order, so the result does not depend
 * on the thread count. */
int oracle_matmul_f64(const uint32_t *w, const void *s, const void *b, int kind,
                      const float *x, double *y, size_t rows, size_t cols, uint32_t bits,
                      size_t group, size_t batch, int threads) {
    return oracle_run(w, s, b, kind, x, y, rows, cols, bits, group, batch, threads, 1);
}

int oracle_matmul_f32(const uint32_t *w, const void *s, const void *b, int kind,
                      const float *x, float *y, size_t rows, size_t cols, uint32_t bits,
                      size_t group, size_t batch, int threads) {
    return oracle_run(w, s, b, kind, x, y, rows, cols, bits, group, batch, threads, 0);
}

/* src/gpu/metadata.rs:6-14: compact only if every value is finite and has
 * zero low 16 bits. Returns 1 and fills out[] when compacted, else 0. */
int oracle_pack_bf16_exact(const float *v, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t bits;
        memcpy(&bits, &v[i], 4);
        if ((bits & 0x7f800000u) == 0x7f800000u || (bits & 0xffffu) != 0) return 0;
    }
    for (size_t i = 0; i < n; ++i) {
        uint32_t bits;
        memcpy(&bits, &v[i], 4);
        out[i] = (uint16_t)(bits >> 16);
    }
    return 1;
}

/* Dense F16 block oracle (tests/batch_matrix.rs:150-160): f16 weights
 * [rows][cols] times token-major x, FP64 accumulate. */
int oracle_dense_f16_f64(const uint16_t *w, const float *x, double *y, size_t rows,
                         size_t cols, size_t batch) {
    if (rows == 0 || cols == 0 || batch == 0) return -1;
    for (size_t t = 0; t < batch; ++t)
        for (size_t r = 0; r < rows; ++r) {
            double acc = 0.0;
            for (size_t c = 0; c < cols; ++c)
                acc += (double)oracle_f16_to_f32(w[r * cols + c]) * (double)x[t * cols + c];
            y[t * rows + r] = acc;
        }
    return 0;
}

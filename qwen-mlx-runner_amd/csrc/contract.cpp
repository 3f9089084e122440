// Host-side dispatch contract (see contract.hpp). Every routine restates the
// reference's host validation or routing so that malformed views and shapes
// are rejected before any device work, with the reference's messages.
#include "contract.hpp"

#include <climits>
#include <cmath>
#include <cstring>

namespace qmr {

namespace {

[[noreturn]] void fail(const std::string &message) { throw Error{1, message}; }

void ensure(bool ok, const std::string &message) {
    if (!ok) fail(message);
}

bool mul_overflow(size_t a, size_t b, size_t *out) { return __builtin_mul_overflow(a, b, out); }

}  // namespace

bool starts_with(const std::string &s, const char *prefix) {
    return s.compare(0, std::strlen(prefix), prefix) == 0;
}

bool ends_with(const std::string &s, const char *suffix) {
    size_t n = std::strlen(suffix);
    return s.size() >= n && s.compare(s.size() - n, n, suffix) == 0;
}

Meta meta_of_name(const std::string &name) {
    if (ends_with(name, "_bf16")) return Meta::BF16;
    if (ends_with(name, "_f16meta")) return Meta::F16;
    return Meta::F32;
}

bool is_wide_name(const std::string &name) { return starts_with(name, "matmul_affine_wide"); }

bool is_block_name(const std::string &name) { return starts_with(name, "matmul_"); }

bool is_residual_name(const std::string &name) {
    return name == "matmul_affine_add" || name == "matmul_affine_add_bf16" || name == "matmul_affine_add_f16meta";
}

bool is_mlp_name(const std::string &name) {
    return name == "mlp_gate_up_swiglu" || name == "mlp_gate_up_swiglu_bf16" || name == "mlp_gate_up_swiglu_f16meta";
}

bool is_fused_name(const std::string &name) { return is_residual_name(name) || is_mlp_name(name); }

bool is_affine_matrix_name(const std::string &name) {
    return starts_with(name, "matvec_affine") || starts_with(name, "matmul_affine");
}

// src/gpu/metadata.rs:16-18.
bool supported_bf16_quantization(uint32_t bits, size_t group) {
    return (bits == 4 || bits == 8) && (group == 32 || group == 64 || group == 128);
}

// src/gpu/metadata.rs:6-14: lossless only if every value is finite with zero
// low 16 bits; keeps signed zeros and BF16 subnormals.
bool pack_bf16_exact(const float *values, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t bits;
        std::memcpy(&bits, &values[i], 4);
        if ((bits & 0x7f800000u) == 0x7f800000u || (bits & 0xffffu) != 0) return false;
    }
    for (size_t i = 0; i < n; ++i) {
        uint32_t bits;
        std::memcpy(&bits, &values[i], 4);
        out[i] = static_cast<uint16_t>(bits >> 16);
    }
    return true;
}

// src/gpu.rs:879-889.
void checked_buffer_range(size_t offset, size_t minimum, size_t length) {
    ensure(offset % 4 == 0, "GPU buffer offsets must be 4-byte aligned");
    size_t end;
    ensure(!__builtin_add_overflow(offset, minimum, &end), "GPU buffer view byte range overflow");
    ensure(end <= length, "GPU buffer view ends at " + std::to_string(end) +
                              " bytes but buffer has " + std::to_string(length));
}

// src/gpu.rs:891-894. Views were overflow-checked first.
bool ranges_overlap(size_t a, size_t a_len, size_t b, size_t b_len) {
    return a < b + b_len && b < a + a_len;
}

// dispatch_layout, matrix part (src/gpu.rs:1041-1172), plus this library's
// F16-metadata and wide-block names.
Layout dispatch_layout(const std::string &name, const uint32_t *p, size_t np) {
    size_t count;
    if (name == "copy_f32") {
        count = 1;
    } else if (name == "read_checksum") {
        count = 3;
    } else if (name == "matvec_f16" || name == "embed_f16") {
        count = 2;
    } else if (name == "matvec_affine" || name == "embed_affine" || name == "matvec_affine_bf16" ||
               name == "embed_affine_bf16" || name == "matvec_affine_f16meta" ||
               name == "embed_affine_f16meta") {
        count = 4;
    } else if (name == "matmul_f16") {
        count = 3;
    } else if (name == "matmul_affine" || name == "matmul_affine_bf16" ||
               name == "matmul_affine_f16meta" || name == "matmul_affine_wide" ||
               name == "matmul_affine_wide_bf16" || is_residual_name(name)) {
        count = 5;
    } else if (is_mlp_name(name)) {
        count = 6;
    } else {
        fail("Unknown GPU kernel " + name);
    }
    ensure(np == count, name + ": expected " + std::to_string(count) + " parameters");
    auto n = [&](size_t i) -> size_t { return p[i]; };
    auto product = [&](std::initializer_list<size_t> v) -> size_t {
        size_t size = 1;
        for (size_t b : v) ensure(!mul_overflow(size, b, &size), "GPU shape overflow");
        ensure(size <= UINT32_MAX, "GPU element index overflow");
        return size;
    };
    auto f = [&](size_t elements) -> size_t {
        size_t bytes;
        ensure(!mul_overflow(elements, 4, &bytes), "GPU byte size overflow");
        return bytes;
    };
    auto positive = [&](std::initializer_list<size_t> idx) {
        for (size_t i : idx) ensure(p[i] > 0, name + ": dimensions must be nonzero");
    };
    const Meta meta = meta_of_name(name);
    const size_t meta_bytes_per = meta == Meta::F32 ? 4 : 2;
    Layout out;

    // read_checksum [a, b, c] (byte sizes, multiples of 4, not all zero) ->
    // views of a, b and c bytes and the checksum slots; one thread per 16
    // bytes read. A library addition: the read floor of the GEMV's bytes.
    if (name == "read_checksum") {
        size_t total = 0;
        for (size_t i = 0; i < 3; ++i) {
            ensure(p[i] % 4 == 0, name + ": view sizes must be multiples of 4 bytes");
            total += p[i];
        }
        ensure(total > 0, name + ": dimensions must be nonzero");
        out.sizes = {n(0), n(1), n(2), size_t(kChecksumSlots) * 4};
        out.threads = (total + 15) / 16;
        return out;
    }

    // src/gpu.rs:1173-1176: copy_f32 [n] -> two views of n floats, n threads.
    if (name == "copy_f32") {
        positive({0});
        out.sizes = {f(product({n(0)})), f(product({n(0)}))};
        out.threads = n(0);
        return out;
    }

    if (starts_with(name, "matvec_") || starts_with(name, "embed_")) {
        positive({1});
        const bool embedding = starts_with(name, "embed");
        size_t rows;
        if (embedding) {
            ensure(n(0) < SIZE_MAX, "Embedding row overflow");
            rows = n(0) + 1;
        } else {
            positive({0});
            rows = n(0);
        }
        const size_t total = product({rows, n(1)});
        const size_t output = embedding ? n(1) : n(0);
        if (ends_with(name, "affine") || meta != Meta::F32) {
            ensure((p[2] == 4 || p[2] == 8) && p[3] > 0,
                   "Only affine 4/8-bit quantization supported");
            ensure(n(1) % (32 / n(2)) == 0 && n(1) % n(3) == 0, "Invalid packed matrix alignment");
            ensure(meta != Meta::BF16 || supported_bf16_quantization(p[2], n(3)),
                   "BF16 metadata supports only affine Q4/Q8 groups 32, 64 or 128");
            ensure(meta != Meta::F16 || supported_bf16_quantization(p[2], n(3)),
                   "F16 metadata supports only affine Q4/Q8 groups 32, 64 or 128");
            size_t metadata_bytes, packed_bits;
            ensure(!mul_overflow(total / n(3), meta_bytes_per, &metadata_bytes),
                   "Affine metadata byte size overflow");
            ensure(!mul_overflow(total, n(2), &packed_bits), "Packed byte size overflow");
            out.sizes = {packed_bits / 8, metadata_bytes, metadata_bytes};
        } else {
            size_t dense;
            ensure(!mul_overflow(total, 2, &dense), "Dense byte size overflow");
            out.sizes = {dense};
        }
        if (!embedding) out.sizes.push_back(f(n(1)));
        out.sizes.push_back(f(output));
        out.threads = embedding ? output : product({output, 32});
        return out;
    }

    // Fused MLP (no reference counterpart): [rows, cols, bits, group, batch,
    // eps bits]; buffers gate w/s/b, up w/s/b, x [batch][cols], RMS-norm
    // weights [cols], y [batch][rows].
    if (is_mlp_name(name)) {
        positive({0, 1});
        const size_t batch = n(4);
        ensure(batch >= 1 && batch <= 4, "Matrix blocks support one through four RHS");
        const float eps = [&] {
            float v;
            std::memcpy(&v, &p[5], 4);
            return v;
        }();
        ensure(std::isfinite(eps) && eps > 0.f, name + ": epsilon must be finite and positive");
        ensure(supported_bf16_quantization(p[2], n(3)), "Matrix blocks support affine Q4/Q8 groups 32, 64 or 128");
        ensure(n(1) % n(3) == 0, "Invalid packed matrix alignment");
        const size_t total = product({n(0), n(1)});
        size_t metadata, packed_bits;
        ensure(!mul_overflow(total / n(3), meta_bytes_per, &metadata), "Affine block metadata byte size overflow");
        ensure(!mul_overflow(total, n(2), &packed_bits), "Packed block byte size overflow");
        out.sizes = {packed_bits / 8, metadata, metadata, packed_bits / 8, metadata, metadata,
                     f(product({batch, n(1)})), f(n(1)), f(product({batch, n(0)}))};
        out.threads = product({n(0), 32});
        return out;
    }

    // Blocks: matmul_affine*, matmul_f16 (src/gpu.rs:1130-1172).
    positive({0, 1});
    const bool affine = name != "matmul_f16";
    const size_t batch = n(affine ? 4 : 2);
    if (is_wide_name(name)) {
        ensure(batch >= 1 && batch <= 256, "Wide matrix blocks support one through 256 RHS");
    } else {
        ensure(batch >= 1 && batch <= 4, "Matrix blocks support one through four RHS");
    }
    const size_t total = product({n(0), n(1)});
    if (affine) {
        ensure(supported_bf16_quantization(p[2], n(3)),
               "Matrix blocks support affine Q4/Q8 groups 32, 64 or 128");
        ensure(n(1) % (32 / n(2)) == 0 && n(1) % n(3) == 0, "Invalid packed matrix alignment");
        size_t metadata, packed_bits;
        ensure(!mul_overflow(total / n(3), meta_bytes_per, &metadata),
               "Affine block metadata byte size overflow");
        ensure(!mul_overflow(total, n(2), &packed_bits), "Packed block byte size overflow");
        out.sizes = {packed_bits / 8, metadata, metadata};
    } else {
        size_t dense;
        ensure(!mul_overflow(total, 2, &dense), "Dense block byte size overflow");
        out.sizes = {dense};
    }
    out.sizes.push_back(f(product({batch, n(1)})));
    if (is_residual_name(name)) out.sizes.push_back(f(product({batch, n(0)})));  // residual r
    out.sizes.push_back(f(product({batch, n(0)})));
    out.threads = product({n(0), 32});
    return out;
}

// specialized_matmul (src/gpu.rs:896-999). Returns the reference pipeline
// name the Metal backend would select; this library maps each to a HIP
// instance. The reference's table is reproduced by construction from its
// (bits, group, batch, metadata) key.
const char *specialized_matmul(const std::string &name, const uint32_t *p, bool aligned,
                               BlockMatmulMode mode) {
    static const char *const dense[] = {"matmul_f16_b1", "matmul_f16_b2", "matmul_f16_b3",
                                        "matmul_f16_b4"};
    if (name == "matmul_f16") {
        if (p[2] >= 1 && p[2] <= 4) return dense[p[2] - 1];
        return nullptr;
    }
    const bool bf16 = ends_with(name, "_bf16");
    if (aligned && p[0] % 4 == 0 && p[1] % 512 == 0 && p[2] == 4 && p[3] == 64 &&
        uint64_t(p[0]) * uint64_t(p[1]) <= uint64_t(INT32_MAX) &&
        uint64_t(p[1]) * uint64_t(p[4]) <= uint64_t(INT32_MAX)) {
        if (mode == BlockMatmulMode::MlpR2 && name == "matmul_affine_bf16" && p[4] == 3 &&
            ((p[0] == 17408 && p[1] == 5120) || (p[0] == 5120 && p[1] == 17408))) {
            return "matmul_q4_g64_b3_mlp_r2_aligned_bf16";
        }
        if (mode == BlockMatmulMode::Shared) {
            if (p[4] == 2) return bf16 ? "matmul_q4_g64_b2_shared_aligned_bf16"
                                       : "matmul_q4_g64_b2_shared_aligned";
            if (p[4] == 3) return bf16 ? "matmul_q4_g64_b3_shared_aligned_bf16"
                                       : "matmul_q4_g64_b3_shared_aligned";
        }
        static const char *const al[4][2] = {
            {"matmul_q4_g64_b1_aligned", "matmul_q4_g64_b1_aligned_bf16"},
            {"matmul_q4_g64_b2_aligned", "matmul_q4_g64_b2_aligned_bf16"},
            {"matmul_q4_g64_b3_aligned", "matmul_q4_g64_b3_aligned_bf16"},
            {"matmul_q4_g64_b4_aligned", "matmul_q4_g64_b4_aligned_bf16"}};
        if (p[4] >= 1 && p[4] <= 4) return al[p[4] - 1][bf16 ? 1 : 0];
        return nullptr;
    }
    // Generic block table, keyed by (bits, group, batch, metadata).
    static const char *const generic[2][3][4][2] = {
        {{{"matmul_q4_g32_b1", "matmul_q4_g32_b1_bf16"},
          {"matmul_q4_g32_b2", "matmul_q4_g32_b2_bf16"},
          {"matmul_q4_g32_b3", "matmul_q4_g32_b3_bf16"},
          {"matmul_q4_g32_b4", "matmul_q4_g32_b4_bf16"}},
         {{"matmul_q4_g64_b1", "matmul_q4_g64_b1_bf16"},
          {"matmul_q4_g64_b2", "matmul_q4_g64_b2_bf16"},
          {"matmul_q4_g64_b3", "matmul_q4_g64_b3_bf16"},
          {"matmul_q4_g64_b4", "matmul_q4_g64_b4_bf16"}},
         {{"matmul_q4_g128_b1", "matmul_q4_g128_b1_bf16"},
          {"matmul_q4_g128_b2", "matmul_q4_g128_b2_bf16"},
          {"matmul_q4_g128_b3", "matmul_q4_g128_b3_bf16"},
          {"matmul_q4_g128_b4", "matmul_q4_g128_b4_bf16"}}},
        {{{"matmul_q8_g32_b1", "matmul_q8_g32_b1_bf16"},
          {"matmul_q8_g32_b2", "matmul_q8_g32_b2_bf16"},
          {"matmul_q8_g32_b3", "matmul_q8_g32_b3_bf16"},
          {"matmul_q8_g32_b4", "matmul_q8_g32_b4_bf16"}},
         {{"matmul_q8_g64_b1", "matmul_q8_g64_b1_bf16"},
          {"matmul_q8_g64_b2", "matmul_q8_g64_b2_bf16"},
          {"matmul_q8_g64_b3", "matmul_q8_g64_b3_bf16"},
          {"matmul_q8_g64_b4", "matmul_q8_g64_b4_bf16"}},
         {{"matmul_q8_g128_b1", "matmul_q8_g128_b1_bf16"},
          {"matmul_q8_g128_b2", "matmul_q8_g128_b2_bf16"},
          {"matmul_q8_g128_b3", "matmul_q8_g128_b3_bf16"},
          {"matmul_q8_g128_b4", "matmul_q8_g128_b4_bf16"}}}};
    int bi = p[2] == 4 ? 0 : p[2] == 8 ? 1 : -1;
    int gi = p[3] == 32 ? 0 : p[3] == 64 ? 1 : p[3] == 128 ? 2 : -1;
    if (bi < 0 || gi < 0 || p[4] < 1 || p[4] > 4) return nullptr;
    return generic[bi][gi][p[4] - 1][bf16 ? 1 : 0];
}

// specialized_matvec (src/gpu.rs:1003-1020).
const char *specialized_matvec(const uint32_t *p, bool aligned) {
    aligned = aligned && p[0] % 4 == 0 && p[1] % 512 == 0 &&
              uint64_t(p[0]) * uint64_t(p[1]) <= uint64_t(INT32_MAX);
    if (p[2] == 4) {
        if (p[3] == 32) return aligned ? "matvec_q4_g32_aligned" : "matvec_q4_g32";
        if (p[3] == 64) return aligned ? "matvec_q4_g64_aligned" : "matvec_q4_g64";
        if (p[3] == 128) return aligned ? "matvec_q4_g128_aligned" : "matvec_q4_g128";
    } else if (p[2] == 8) {
        if (p[3] == 32) return "matvec_q8_g32";
        if (p[3] == 64) return "matvec_q8_g64";
        if (p[3] == 128) return "matvec_q8_g128";
    }
    return nullptr;
}

// specialized_matvec_bf16 (src/gpu.rs:1022-1037).
const char *specialized_matvec_bf16(const uint32_t *p, bool aligned) {
    aligned = aligned && p[0] % 4 == 0 && p[1] % 512 == 0 &&
              uint64_t(p[0]) * uint64_t(p[1]) <= uint64_t(INT32_MAX);
    if (p[2] == 4) {
        if (p[3] == 64 && aligned) return "matvec_q4_g64_aligned_bf16";
        if (p[3] == 32) return "matvec_q4_g32_bf16";
        if (p[3] == 64) return "matvec_q4_g64_bf16";
        if (p[3] == 128) return "matvec_q4_g128_bf16";
    } else if (p[2] == 8) {
        if (p[3] == 32) return "matvec_q8_g32_bf16";
        if (p[3] == 64) return "matvec_q8_g64_bf16";
        if (p[3] == 128) return "matvec_q8_g128_bf16";
    }
    return nullptr;
}

// BlockKernelMode::parse (src/gpu.rs:62-77). Exact, case-sensitive strings.
BlockKernelMode parse_block_kernel_mode(const char *matmul, const char *delta) {
    BlockKernelMode mode;
    std::string m = matmul ? matmul : "legacy";
    std::string d = delta ? delta : "batched";
    if (m == "legacy") {
        mode.matmul = BlockMatmulMode::Legacy;
    } else if (m == "shared") {
        mode.matmul = BlockMatmulMode::Shared;
    } else if (m == "mlp-r2") {
        mode.matmul = BlockMatmulMode::MlpR2;
    } else {
        fail("QWEN_METAL_BLOCK_MATMUL must be legacy, shared or mlp-r2");
    }
    ensure(d == "sequential" || d == "batched",
           "QWEN_METAL_BLOCK_DELTA must be sequential or batched");
    mode.batched_delta = d == "batched";
    return mode;
}

// BlockKernelMode::parse_for_device (src/gpu.rs:49-61). The reference enables
// the R2 schedule by default only on the one device it measured it on; on
// every other device name (this backend's included) Legacy is the default.
BlockKernelMode parse_block_kernel_mode_for_device(const std::string &device_name,
                                                   const char *matmul, const char *delta) {
    const char *def = device_name == "Apple M5 Pro" ? "mlp-r2" : "legacy";
    return parse_block_kernel_mode(matmul ? matmul : def, delta ? delta : "batched");
}

}  // namespace qmr

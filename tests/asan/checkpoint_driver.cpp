// Host-only driver of the checkpoint loader for AddressSanitizer runs
// (tests/test_checkpoint_asan.py): opens each directory given on the command
// line and reads every matrix name that follows "--" through the C ABI. The
// device-facing entry points the loader calls are stubbed: this exercises
// parsing, validation and value decoding, not uploads.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/qmr_checkpoint.h"
#include "../../qwen-mlx-runner_amd/csrc/contract.hpp"

static std::string g_error;
namespace qmr {
int record_error(int code, const std::string &message) {
    g_error = message;
    return code;
}
void clear_error() { g_error.clear(); }
size_t device_free_bytes(const ::qmr_device *) { return 0; }
int upload_staged(::qmr_device *, const void *, size_t, ::qmr_buffer **) { return QMR_ERR_DEVICE; }
int upload_staged_views(::qmr_device *, const StagedView *, size_t, ::qmr_buffer **) { return QMR_ERR_DEVICE; }
}  // namespace qmr
extern "C" {
const char *qmr_last_error(void) { return g_error.c_str(); }
int qmr_buffer_upload(qmr_device *, const void *, size_t, qmr_buffer **) { return QMR_ERR_DEVICE; }
void qmr_buffer_release(qmr_buffer *) {}
const char *qmr_metadata_mode(const qmr_device *) { return "f32"; }
int qmr_supported_bf16_quantization(uint32_t bits, size_t group) {
    return qmr::supported_bf16_quantization(bits, group) ? 1 : 0;
}
int qmr_compact_metadata(const qmr_device *, uint32_t, size_t, const float *, const float *, size_t, uint16_t *,
                         uint16_t *) {
    return 0;
}
void qmr_record_compacted_metadata(qmr_device *, uint64_t) {}
}

int main(int argc, char **argv) {
    std::vector<std::string> dirs, names;
    bool after = false;
    for (int i = 1; i < argc; ++i) {
        if (!std::strcmp(argv[i], "--")) after = true;
        else (after ? names : dirs).push_back(argv[i]);
    }
    size_t opened = 0, read = 0;
    for (const auto &d : dirs) {
        qmr_checkpoint *cp = nullptr;
        if (qmr_checkpoint_open(d.c_str(), &cp) != QMR_OK) continue;
        ++opened;
        for (const auto &n : names) {
            qmr_matrix_info info;
            if (qmr_checkpoint_matrix_info(cp, n.c_str(), &info) != QMR_OK) continue;
            if (info.rows > (1u << 20) || info.cols > (1u << 20)) continue;
            if (info.packed) {
                std::vector<uint32_t> w(info.rows * info.cols / (32 / info.bits));
                std::vector<float> s(info.rows * info.cols / info.group_size), b(s.size());
                if (qmr_checkpoint_matrix(cp, n.c_str(), w.data(), s.data(), b.data()) == QMR_OK) ++read;
            } else {
                std::vector<uint16_t> v(info.rows * info.cols);
                if (qmr_checkpoint_dense(cp, n.c_str(), v.data()) == QMR_OK) ++read;
            }
            qmr_matrix m;
            qmr_matrix_load(reinterpret_cast<qmr_device *>(&m), cp, n.c_str(), info.rows, info.cols, &m);
        }
        qmr_checkpoint_close(cp);
    }
    std::printf("opened %zu read %zu\n", opened, read);
    return 0;
}

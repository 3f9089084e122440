// Host runtime behind include/qmr.h: device, buffers, commands and the
// checked dispatch path. Replaces the reference's Metal backend object model
// (Gpu / DispatchEncoder / command buffers, src/gpu.rs:95-876) with HIP:
// one stream per device, asynchronous launches, one synchronisation per
// command at qmr_command_finish.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "../../include/qmr.h"
#include "contract.hpp"
#include "kernels.hpp"

using qmr::Error;

// Everything a row-band plan depends on: rows, cols, bits, group, batch,
// metadata format, MLP form, residual form, forced plan code, block schedule.
using BandPlanKey = std::tuple<uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, int, bool, bool, int, int>;

// Scratch of the no-allocation entry point (qmr_encode_static): a fixed array
// in the code object, so that every GPU the library runs on holds its own
// copy from module load until the process ends. On the host the array's name
// is not a device address: host code reaches a GPU's copy only through the
// address hipGetSymbolAddress returns with that GPU current (scratch_entry
// below, kept in qmr_device::scratch). Every qmr_encode_static call on a GPU
// shares its copy, which keeps the last call's contents.
static __device__ __align__(256) unsigned char scratch[QMR_STATIC_SCRATCH_BYTES];

struct qmr_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    std::string name;
    std::string gemv_variant = "aligned";
    bool reference = false;
    bool bf16_metadata = false;
    qmr::BlockKernelMode block_mode;
    size_t max_alloc = 0;
    qmr::DeviceLimits limits{};
    size_t compacted_matrices = 0;
    uint64_t metadata_saved_bytes = 0;
    // Testing/tuning hook; {0,0} = planner. rr = -3: row-owning matrix-core
    // kernel, opt-in (ks = j*10000 + rt*100 + kw; j = 0 or ks = 0 leave the
    // choice to its planner); rr = -2: split-K matrix-core kernel; rr = -1 or
    // rr > 0: vector-ALU kernels.
    qmr::GemvPlan forced_plan;
    std::string last_kernel;    // selected reference pipeline label
    std::string last_hip;       // HIP kernel (and plan) of the last launch
    // Per-band arrival counters of the split-K matrix-core kernel (kept zero
    // between launches).
    uint32_t *ws_counters = nullptr;
    size_t ws_counter_count = 0;
    // Workspace of the row-band and split-K kernels' partial sums: 64-bit
    // {value, epoch} slots (contents need no clearing: a slot counts only
    // when its epoch is the launch's), and the epoch of the last launch.
    unsigned long long *ws_slots = nullptr;
    size_t ws_slots_bytes = 0;
    uint32_t slot_epoch = 0;
    // Row-band plans by shape, format, form, forced plan and block schedule:
    // planning enumerates ~100 shapes with occupancy queries, which must not
    // sit on every launch.
    mutable std::map<BandPlanKey, qmr::TilePlan> band_plans;
    // Dense matrix-core plans by rows, cols, batch and forced plan (-1: the
    // default choice).
    mutable std::map<std::tuple<uint32_t, uint32_t, uint32_t, int>, qmr::DensePlan> dense_plans;
    // Workspace of the wide-block kernel: the activation images.
    unsigned char *ws_wide = nullptr;
    size_t ws_wide_bytes = 0;
    // This GPU's copy of the static scratch (the workspace of
    // qmr_encode_static, which allocates nothing), and how many of its
    // leading bytes may be non-zero (shared by every handle on the GPU).
    unsigned char *scratch = nullptr;
    std::atomic<size_t> *scratch_dirty = nullptr;
    // Status word the row-band kernel sets when a last split gives up
    // (host-coherent memory mapped into the device; read at finish), and its
    // device address.
    uint32_t *status_host = nullptr;
    uint32_t *status_dev = nullptr;
    // Testing hook: the row-band kernel's last splits give up (qmr_set_band_wait_fault).
    bool force_give_up = false;
    // Tuning hook: read_checksum's geometry (qmr_set_read_plan).
    qmr::ReadPlan read_plan;
    // The open command whose start event is not recorded yet: it is recorded
    // on the stream just before the command's first launch (after any
    // workspace growth), so that a frame's GPU time starts when its GPU work
    // can start, not when the host began encoding.
    qmr_command *pending = nullptr;
    // Pinned staging slots of qmr::upload_staged_views (allocated on first use).
    void *pin[qmr::kStageSlots] = {};
    hipEvent_t pin_done[qmr::kStageSlots] = {};
};

struct qmr_buffer {
    int ordinal = 0;
    void *ptr = nullptr;
    size_t length = 0;
    std::atomic<int> refs{1};
};

struct qmr_command {
    qmr_device *device = nullptr;
    std::chrono::steady_clock::time_point started;
    // marks[0] = GPU start (recorded before the first launch, or at finish
    // when nothing was launched); finish appends the end.
    std::vector<hipEvent_t> marks;
    bool start_recorded = false;
    bool finished = false;
    int end_mark = -1;
};

namespace {

thread_local std::string g_error;

int set_error(int code, const std::string &message) {
    g_error = message;
    return code;
}

int hip_error(hipError_t e, const char *what) {
    return set_error(QMR_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

template <typename F>
int guarded(F &&f) {
    try {
        g_error.clear();
        return f();
    } catch (const Error &e) {
        return set_error(e.code, e.message);
    } catch (const std::exception &e) {
        return set_error(QMR_ERR_INVALID, e.what());
    }
}

void ensure(bool ok, const std::string &message, int code = QMR_ERR_INVALID) {
    if (!ok) throw Error{code, message};
}

void check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess) throw Error{QMR_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e)};
}

// Records a command's start event on its device's stream (once).
void record_start(qmr_command *cmd) {
    if (cmd->start_recorded) return;
    if (cmd->device->pending == cmd) cmd->device->pending = nullptr;
    check_hip(hipEventRecord(cmd->marks[0], cmd->device->stream), "hipEventRecord");
    cmd->start_recorded = true;
}

// Records the open command's start event if it is still pending: called by
// every launch path right before its first launch, after workspace growth.
void start_gpu(qmr_device *dev) {
    if (dev->pending) record_start(dev->pending);
}

}  // namespace

namespace qmr {
int record_error(int code, const std::string &message) { return set_error(code, message); }
void clear_error() { g_error.clear(); }
}  // namespace qmr

namespace qmr {

namespace {

// Host threads that copy one staging chunk together: each round the caller
// publishes (dst, src, len) and every member copies its share; the crew
// lives for one upload, so its threads start once and not per chunk.
class CopyCrew {
public:
    explicit CopyCrew(unsigned n) : n_(n) {
        try {
            for (unsigned t = 1; t < n_; ++t) threads_.emplace_back([this, t] { run(t); });
        } catch (...) {
            stop();  // threads already started must not outlive a crew that failed to form
            throw;
        }
    }
    ~CopyCrew() { stop(); }
    void copy(unsigned char *dst, const unsigned char *src, size_t len) {
        {
            std::lock_guard<std::mutex> lock(mu_);
            dst_ = dst;
            src_ = src;
            len_ = len;
            pending_ = unsigned(threads_.size());
            ++round_;
        }
        go_.notify_all();
        share(0, dst, src, len);
        std::unique_lock<std::mutex> lock(mu_);
        done_.wait(lock, [&] { return pending_ == 0; });
    }

private:
    void stop() {
        {
            std::lock_guard<std::mutex> lock(mu_);
            quit_ = true;
        }
        go_.notify_all();
        for (auto &t : threads_) t.join();
        threads_.clear();
    }
    void share(unsigned t, unsigned char *dst, const unsigned char *src, size_t len) const {
        const size_t part = (len + n_ - 1) / n_;
        const size_t b = size_t(t) * part;
        if (b < len) std::memcpy(dst + b, src + b, std::min(part, len - b));
    }
    void run(unsigned t) {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lock(mu_);
        for (;;) {
            go_.wait(lock, [&] { return quit_ || round_ != seen; });
            if (quit_) return;
            seen = round_;
            unsigned char *dst = dst_;
            const unsigned char *src = src_;
            const size_t len = len_;
            lock.unlock();
            share(t, dst, src, len);
            lock.lock();
            if (--pending_ == 0) done_.notify_one();
        }
    }
    const unsigned n_;
    std::vector<std::thread> threads_;
    std::mutex mu_;
    std::condition_variable go_, done_;
    uint64_t round_ = 0;
    unsigned pending_ = 0;
    bool quit_ = false;
    unsigned char *dst_ = nullptr;
    const unsigned char *src_ = nullptr;
    size_t len_ = 0;
};

}  // namespace

// Host-to-device copies of pageable sources (mapped checkpoint shards) into
// new device buffers through the device's pinned staging slots: a crew of
// host threads fills one slot with the next chunk while the DMA engine
// drains the others on the device's stream, and the views run through one
// pipeline, so a matrix's codes, scales and biases overlap. Chunks of 8 MB
// over three slots keep the first fill and the last drain short. Measured on
// MI355X (one layer's three MLP matrices, 150 MB): 2.25 ms per matrix with
// two 16 MB slots and one pipeline per array, the arrays uploaded one after
// the other.
int upload_staged_views(::qmr_device *device, const StagedView *views, size_t n, ::qmr_buffer **outs) {
    constexpr size_t kChunk = kStageChunk;
    constexpr unsigned kThreads = 8;
    return guarded([&]() -> int {
        ensure(device && (views || n == 0) && (outs || n == 0), "upload_staged: null argument");
        for (size_t i = 0; i < n; ++i) {
            outs[i] = nullptr;
            ensure(views[i].src != nullptr || views[i].bytes == 0, "upload_staged: null source");
            ensure(views[i].bytes <= device->max_alloc, "GPU allocation " + std::to_string(views[i].bytes) +
                                                            " exceeds device buffer limit " +
                                                            std::to_string(device->max_alloc));
        }
        check_hip(hipSetDevice(device->ordinal), "hipSetDevice");
        for (int i = 0; i < kStageSlots; ++i) {
            if (!device->pin[i]) check_hip(hipHostMalloc(&device->pin[i], kChunk, hipHostMallocDefault), "hipHostMalloc");
            if (!device->pin_done[i])
                check_hip(hipEventCreateWithFlags(&device->pin_done[i], hipEventDisableTiming), "hipEventCreate");
        }
        std::vector<void *> dst(n, nullptr);
        auto free_all = [&] {
            for (void *d : dst)
                if (d) hipFree(d);
        };
        hipError_t e = hipSuccess;
        for (size_t i = 0; i < n && e == hipSuccess; ++i) e = hipMalloc(&dst[i], views[i].bytes > 0 ? views[i].bytes : 4);
        if (e != hipSuccess) {
            free_all();
            check_hip(e, "hipMalloc");
        }
        {
            CopyCrew crew(kThreads);
            size_t k = 0;  // chunks issued, over all views
            for (size_t i = 0; i < n && e == hipSuccess; ++i) {
                const auto *from = static_cast<const unsigned char *>(views[i].src);
                for (size_t pos = 0; pos < views[i].bytes && e == hipSuccess; pos += kChunk, ++k) {
                    const int slot = int(k % kStageSlots);
                    const size_t len = std::min(kChunk, views[i].bytes - pos);
                    // The slot's previous chunk must have landed before it is refilled.
                    if (k >= size_t(kStageSlots)) e = hipEventSynchronize(device->pin_done[slot]);
                    if (e != hipSuccess) break;
                    auto *stage = static_cast<unsigned char *>(device->pin[slot]);
                    crew.copy(stage, from + pos, len);
                    e = hipMemcpyAsync(static_cast<unsigned char *>(dst[i]) + pos, stage, len, hipMemcpyHostToDevice,
                                       device->stream);
                    if (e == hipSuccess) e = hipEventRecord(device->pin_done[slot], device->stream);
                }
            }
        }
        if (e == hipSuccess) e = hipStreamSynchronize(device->stream);
        if (e != hipSuccess) {
            hipStreamSynchronize(device->stream);
            free_all();
            check_hip(e, "staged upload");
        }
        for (size_t i = 0; i < n; ++i) {
            auto *b = new ::qmr_buffer();
            b->ordinal = device->ordinal;
            b->ptr = dst[i];
            b->length = views[i].bytes;
            outs[i] = b;
        }
        return QMR_OK;
    });
}

int upload_staged(::qmr_device *device, const void *src, size_t bytes, ::qmr_buffer **out) {
    const StagedView v{src, bytes};
    return upload_staged_views(device, &v, 1, out);
}

hipError_t raise_lds_limit(const void *kernel, size_t bytes) {
    static std::mutex mu;
    static std::vector<std::pair<std::pair<const void *, int>, size_t>> done;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    for (auto &d : done) {
        if (d.first.first != kernel || d.first.second != dev) continue;
        if (d.second >= bytes) return hipSuccess;
        e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
        if (e == hipSuccess) d.second = bytes;
        return e;
    }
    e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
    if (e == hipSuccess) done.push_back({{kernel, dev}, bytes});
    return e;
}

size_t device_free_bytes(const ::qmr_device *device) {
    size_t free_bytes = 0, total = 0;
    check_hip(hipSetDevice(device->ordinal), "hipSetDevice");
    check_hip(hipMemGetInfo(&free_bytes, &total), "hipMemGetInfo");
    return free_bytes;
}
}  // namespace qmr

namespace {

bool is_variant(const std::string &v) {
    return v == "packed4" || v == "aligned" || v == "stream";
}

// Upper bound of threads a reference pipeline accepts per threadgroup: the
// aligned/stream pipelines are built with 64, the other specialised matrix
// pipelines with 128 (src/gpu.rs:394-414); generic ones keep the default.
size_t pipeline_max_threads(const char *label) {
    if (!label) return 1024;
    std::string n = label;
    if (qmr::ends_with(n, "_aligned") || qmr::ends_with(n, "_aligned_bf16") ||
        qmr::ends_with(n, "_stream"))
        return 64;
    if (qmr::starts_with(n, "matvec_q") || qmr::starts_with(n, "matmul_")) return 128;
    return 1024;
}

// The device address of `scratch` on GPU `ordinal`, looked up once per GPU
// with that GPU current (the caller has made it current) and kept for the
// process, like the array itself; with it, the GPU's count of the scratch's
// leading bytes that may be non-zero (all of it until a fill kernel has
// cleared it), shared by every device handle on that GPU.
struct ScratchEntry {
    unsigned char *address;
    std::atomic<size_t> *dirty;
};
ScratchEntry scratch_entry(int ordinal) {
    static std::mutex mu;
    static std::unordered_map<int, ScratchEntry> entries;
    std::lock_guard<std::mutex> lock(mu);
    const auto it = entries.find(ordinal);
    if (it != entries.end()) return it->second;
    void *p = nullptr;
    check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress (static scratch)");
    ensure(p != nullptr, "hipGetSymbolAddress returned no address for the static scratch", QMR_ERR_DEVICE);
    const ScratchEntry e{static_cast<unsigned char *>(p), new std::atomic<size_t>(QMR_STATIC_SCRATCH_BYTES)};
    entries.emplace(ordinal, e);
    return e;
}

// qmr_encode_static runs only launches whose workspace fits the static
// scratch; larger ones are rejected before anything is enqueued.
void check_static_scratch(size_t need, const char *what) {
    ensure(need <= QMR_STATIC_SCRATCH_BYTES,
           std::string("qmr_encode_static: the ") + what + " need " + std::to_string(need) +
               " bytes of scratch; the static scratch holds " + std::to_string(QMR_STATIC_SCRATCH_BYTES) +
               " (use qmr_encode, which grows its workspace)");
}

// The static scratch's first `need` bytes, zeroed for a launch that tags its
// slots with epoch 1: a fill kernel (so that a captured graph clears them on
// every replay) clears everything earlier launches may have left non-zero.
hipError_t clear_static_slots(qmr_device *dev, unsigned char *fixed, size_t need) {
    const size_t dirty = dev->scratch_dirty->load();
    if (need == 0 || dirty == 0) return hipSuccess;
    const size_t n = (need > dirty ? need : dirty) / 4;
    const hipError_t e = qmr::launch_zero_u32(reinterpret_cast<uint32_t *>(fixed), uint32_t(n), dev->stream);
    if (e == hipSuccess) dev->scratch_dirty->store(0);
    return e;
}

// Record that a launch may have left the static scratch's first `extent`
// bytes non-zero.
void mark_static_dirty(qmr_device *dev, size_t extent) {
    size_t cur = dev->scratch_dirty->load();
    while (cur < extent && !dev->scratch_dirty->compare_exchange_weak(cur, extent)) {
    }
}

// The device's slot workspace, grown to `need` bytes (after the stream
// drains, since queued launches may use the old one), and the epoch of a new
// launch that uses it. When the epoch wraps, the slots are cleared so that no
// stale slot can carry the new epoch.
uint32_t next_slot_epoch(qmr_device *dev, size_t need) {
    if (need > dev->ws_slots_bytes) {
        check_hip(hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
        if (dev->ws_slots) hipFree(dev->ws_slots);
        dev->ws_slots = nullptr;
        dev->ws_slots_bytes = 0;
        const size_t n = need < (size_t(1) << 20) ? (size_t(1) << 20) : need;
        check_hip(hipMalloc(&dev->ws_slots, n), "hipMalloc (slot workspace)");
        check_hip(hipMemsetAsync(dev->ws_slots, 0, n, dev->stream), "hipMemsetAsync (slot workspace)");
        dev->ws_slots_bytes = n;
    }
    if (++dev->slot_epoch == 0) {
        if (dev->ws_slots)
            check_hip(hipMemsetAsync(dev->ws_slots, 0, dev->ws_slots_bytes, dev->stream),
                      "hipMemsetAsync (slot workspace)");
        dev->slot_epoch = 1;
    }
    return dev->slot_epoch;
}

// Grow the split-K arrival counters (synchronising the stream before an old
// buffer is freed, since queued launches may still use it).
void ensure_counters(qmr_device *dev, size_t counters) {
    if (counters > dev->ws_counter_count) {
        check_hip(hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
        if (dev->ws_counters) hipFree(dev->ws_counters);
        dev->ws_counters = nullptr;
        dev->ws_counter_count = 0;
        size_t n = counters < 4096 ? 4096 : counters;
        check_hip(hipMalloc(&dev->ws_counters, n * sizeof(uint32_t)), "hipMalloc (counters)");
        check_hip(hipMemsetAsync(dev->ws_counters, 0, n * sizeof(uint32_t), dev->stream),
                  "hipMemsetAsync (counters)");
        dev->ws_counter_count = n;
    }
}

// The row-owning kernel's plan, honouring a forced workgroup shape.
qmr::RowsPlan forced_rows_plan(const qmr_device *dev, const qmr::AffineArgs &a) {
    const qmr::GemvPlan f = dev->forced_plan;
    if (f.rr == -3 && f.ks > 0)
        return qmr::plan_affine_rows(a, dev->limits, uint32_t(f.ks / 100 % 100), uint32_t(f.ks % 100),
                                     uint32_t(f.ks / 10000));
    return qmr::plan_affine_rows(a, dev->limits);
}

// Whether the default planner hands a split-K plan to the row-owning kernel.
// Every split-K workgroup pays fixed costs (its metadata staging, the partial
// store and the band's last-arrival sum) that its K range has to amortise.
// They repeat round after round when the grid needs more than one round of
// resident workgroups (tall matrices such as a vocabulary head), and they
// dominate when a split covers fewer than four K tiles (small matrices, and
// 8-bit codes, whose rows hold few 128-byte entries): measured on MI355X, a
// 5120x5120 Q8 projection takes 9-10 us on the row-owning kernel against
// 11.9 us split 14 ways over 3-tile splits, while the MLP shapes (8-tile
// splits) stay faster split-K.
bool rows_preferred(const qmr::MfmaPlan &pl) {
    return pl.rounds > 1 || (pl.ns > 1 && pl.tps < 4);
}

// The reference's block schedules (src/gpu.rs:22-31) keep each output row's
// accumulation order and change only the thread geometry
// (kernels/matmul_block.metal:291-299). On the row-band kernel the same holds
// for the ring depth and the row tiles per band, which leave a row's sums
// untouched, so the schedules the reference routes to its shared and R2
// pipelines run their own instances: the other ring depth (shared) or half
// (else twice) the row tiles per band (R2), with the splits and waves of the
// legacy plan, and produce its bits.
enum class BandSchedule { Legacy = 0, Shared = 1, R2 = 2 };

BandSchedule band_schedule(const qmr_device *dev) {
    const std::string &label = dev->last_kernel;
    if (qmr::ends_with(label, "_mlp_r2_aligned_bf16")) return BandSchedule::R2;
    if (label.find("_shared_aligned") != std::string::npos) return BandSchedule::Shared;
    return BandSchedule::Legacy;
}

// The row-band kernel's plan, honouring a forced shape (rr == -4, ks =
// ring*100000 + ns*10000 + tr*100 + kw; zero fields leave them to its
// planner) and the block schedule; a schedule's instance that has no
// one-round plan runs the legacy plan. Plans are cached under every field
// they depend on.
qmr::TilePlan forced_tile_plan(const qmr_device *dev, const qmr::AffineArgs &a,
                               BandSchedule sched = BandSchedule::Legacy) {
    const qmr::GemvPlan f = dev->forced_plan;
    const int ks = f.rr == -4 ? f.ks : 0;
    const BandPlanKey key{a.rows, a.cols, a.bits, a.group, a.batch, static_cast<int>(a.meta), a.up_w != nullptr,
                          a.residual != nullptr, ks, static_cast<int>(sched)};
    const auto it = dev->band_plans.find(key);
    if (it != dev->band_plans.end()) return it->second;
    qmr::TilePlan pl = sched != BandSchedule::Legacy ? forced_tile_plan(dev, a)
                       : ks > 0 ? qmr::plan_affine_tile(a, dev->limits, uint32_t(ks % 100), uint32_t(ks / 100 % 100),
                                                        uint32_t(ks / 10000 % 10), uint32_t(ks / 100000 % 10),
                                                        uint32_t(ks / 1000000 % 10))
                                : qmr::plan_affine_tile(a, dev->limits);
    if (pl.kw > 0 && sched == BandSchedule::Shared) {
        const qmr::TilePlan alt = qmr::plan_affine_tile(a, dev->limits, pl.kw, pl.tr, pl.ns, pl.ring == 3 ? 2 : 3);
        if (alt.kw > 0) pl = alt;
    } else if (pl.kw > 0 && sched == BandSchedule::R2) {
        qmr::TilePlan alt;
        if (pl.tr >= 2) alt = qmr::plan_affine_tile(a, dev->limits, pl.kw, pl.tr / 2, pl.ns, pl.ring);
        if (alt.kw == 0 && pl.tr <= 4) alt = qmr::plan_affine_tile(a, dev->limits, pl.kw, pl.tr * 2, pl.ns, pl.ring);
        if (alt.kw > 0) pl = alt;
    }
    if (dev->band_plans.size() > 4096) dev->band_plans.clear();
    dev->band_plans.emplace(key, pl);
    return pl;
}

// Launch the row-band kernel over the device's slot workspace (and, for
// plans with elected finishers, its arrival counters), or with `fixed`
// (qmr_encode_static) over the static scratch: slots, then counters.
hipError_t launch_band(qmr_device *dev, const qmr::AffineArgs &a, const qmr::TilePlan &pl,
                       unsigned char *fixed) {
    const size_t need = qmr::affine_tile_workspace(pl, a);
    const bool elect = pl.elect && pl.ns > 1;
    dev->last_hip = "affine_band_kernel ring=" + std::to_string(pl.ring) + " ns=" + std::to_string(pl.ns) +
                    " tr=" + std::to_string(pl.tr) + " kw=" + std::to_string(pl.kw) + (elect ? " elect" : "") +
                    (pl.phases == 2 ? " phased" : "");
    qmr::TileWait wait;
    wait.status = dev->status_dev;
    wait.force_give_up = dev->force_give_up;
    if (fixed) {
        // The sums are tagged with epoch 1, which no cleared slot carries.
        // The plain and residual forms' finishers clear each slot (and
        // counter) they take, so once the region is zero it stays zero from
        // launch to launch and needs no fill; it is cleared when earlier
        // launches may have left it non-zero: first use on this GPU, after
        // the wide path used the scratch, after an MLP form (whose slots are
        // not cleared) and after a command that failed.
        const size_t part = (need + 255) / 256 * 256;
        const size_t extent = elect ? part + size_t(pl.nbands) * sizeof(uint32_t) : need;
        check_static_scratch(extent, "row-band split sums");
        start_gpu(dev);
        const bool plain = a.up_w == nullptr;
        hipError_t e = clear_static_slots(dev, fixed, (extent + 3) / 4 * 4);
        if (e != hipSuccess) return e;
        wait.reset_slots = plain;
        uint32_t *counters = elect ? reinterpret_cast<uint32_t *>(fixed + part) : nullptr;
        e = qmr::launch_affine_tile(a, pl, reinterpret_cast<unsigned long long *>(fixed), counters, 1u, wait,
                                    dev->stream);
        if (!plain || e != hipSuccess) mark_static_dirty(dev, extent);
        return e;
    }
    const uint32_t epoch = next_slot_epoch(dev, need);
    if (elect) ensure_counters(dev, pl.nbands);
    start_gpu(dev);
    return qmr::launch_affine_tile(a, pl, dev->ws_slots, elect ? dev->ws_counters : nullptr, epoch, wait,
                                   dev->stream);
}

// Launch the split-K kernel with its partial-sum slots and per-band arrival
// counters: the device's workspaces, or with `fixed` (qmr_encode_static) the
// static scratch (slots, then counters), zeroed where earlier launches may
// have left data; its last arrivers clear every slot they take and their
// counters, so a successful launch leaves the region zero.
hipError_t launch_split_k(qmr_device *dev, const qmr::AffineArgs &a, const qmr::MfmaPlan &pl,
                          unsigned char *fixed) {
    qmr::TileWait wait;
    wait.status = dev->status_dev;
    wait.force_give_up = dev->force_give_up;
    const size_t need = qmr::affine_mfma_workspace(pl, a);
    if (!fixed) {
        const uint32_t epoch = next_slot_epoch(dev, need);
        ensure_counters(dev, pl.nbands);
        start_gpu(dev);
        return qmr::launch_affine_mfma(a, pl, dev->ws_slots, dev->ws_counters, epoch, wait, dev->stream);
    }
    const size_t part = (need + 255) / 256 * 256;
    const size_t extent = part + size_t(pl.nbands) * sizeof(uint32_t);
    check_static_scratch(extent, "split-K partial sums and counters");
    uint32_t *counters = reinterpret_cast<uint32_t *>(fixed + part);
    start_gpu(dev);
    hipError_t e = clear_static_slots(dev, fixed, (extent + 3) / 4 * 4);
    if (e != hipSuccess) return e;
    wait.reset_slots = true;
    e = qmr::launch_affine_mfma(a, pl, reinterpret_cast<unsigned long long *>(fixed), counters, 1u, wait,
                                dev->stream);
    if (e != hipSuccess) mark_static_dirty(dev, extent);
    return e;
}

// The dense matrix-core kernel's plan for a view it supports, honouring a
// forced shape (rr == -5, ks = ring*10000 + kw*1000 + rt*100 + ns; zero
// fields leave them to its planner). rt == 0 sends the product to the
// vector-ALU kernels: when the hook asks for them (rr == -1), when the view
// is not supported, and by default for one RHS (where the streaming kernel
// is within 6% of the best matrix-core plan on the decoder's shapes and
// faster on most) or when the planner's estimate is not below the
// vector-ALU kernel's (small matrices, whose fixed costs dominate).
qmr::DensePlan dense_plan(const qmr_device *dev, const uint16_t *w, uint32_t rows, uint32_t cols,
                          uint32_t batch) {
    const qmr::GemvPlan f = dev->forced_plan;
    if (f.rr == -1 || !qmr::dense_mfma_supported(w, rows, cols, batch)) return qmr::DensePlan{};
    if (f.rr != -5 && batch == 1) return qmr::DensePlan{};
    const int ks = f.rr == -5 ? f.ks : 0;
    const auto key = std::make_tuple(rows, cols, batch, f.rr == -5 ? ks : -1);
    const auto it = dev->dense_plans.find(key);
    if (it != dev->dense_plans.end()) return it->second;
    qmr::DenseForce force;
    force.ring = uint32_t(ks / 10000 % 10);
    force.kw = uint32_t(ks / 1000 % 10);
    force.rt = uint32_t(ks / 100 % 10);
    force.ns = uint32_t(ks % 100);
    qmr::DensePlan pl = qmr::plan_dense_mfma(rows, cols, batch, dev->limits, force);
    if (f.rr != -5 && pl.rt > 0 && !(pl.cost_us < qmr::dense_valu_cost(rows, cols, batch))) pl = qmr::DensePlan{};
    if (dev->dense_plans.size() > 4096) dev->dense_plans.clear();
    dev->dense_plans.emplace(key, pl);
    return pl;
}

// Dense F16 matvec / block: the matrix-core kernel where it has a plan
// (its split sums in the device's slot workspace, or with `fixed` in the
// static scratch, whose region its finishers leave zero), else the
// vector-ALU kernels, which need no workspace; so does a static launch
// whose plan's sums would not fit the static scratch.
hipError_t launch_dense(qmr_device *dev, const uint16_t *w, const float *x, float *y, uint32_t rows, uint32_t cols,
                        uint32_t batch, unsigned char *fixed) {
    const qmr::DensePlan pl = dense_plan(dev, w, rows, cols, batch);
    const size_t need = pl.rt > 0 ? qmr::dense_mfma_workspace(pl, rows, batch) : 0;
    const size_t part = (need + 255) / 256 * 256;
    const size_t extent = pl.ns > 1 ? part + size_t(pl.nbands) * sizeof(uint32_t) : 0;
    if (pl.rt == 0 || (fixed && extent > QMR_STATIC_SCRATCH_BYTES)) {
        dev->last_hip = "dense_f16_kernel";
        start_gpu(dev);
        return qmr::launch_dense_f16(w, x, y, rows, cols, batch, dev->stream);
    }
    dev->last_hip = "dense_mfma_kernel ring=" + std::to_string(pl.ring) + " kw=" + std::to_string(pl.kw) +
                    " rt=" + std::to_string(pl.rt) + " ns=" + std::to_string(pl.ns);
    qmr::TileWait wait;
    wait.status = dev->status_dev;
    wait.force_give_up = dev->force_give_up;
    if (pl.ns == 1) {
        start_gpu(dev);
        return qmr::launch_dense_mfma(w, x, y, rows, cols, batch, pl, nullptr, nullptr, 1u, wait, dev->stream);
    }
    if (!fixed) {
        const uint32_t epoch = next_slot_epoch(dev, need);
        ensure_counters(dev, pl.nbands);
        start_gpu(dev);
        return qmr::launch_dense_mfma(w, x, y, rows, cols, batch, pl, dev->ws_slots, dev->ws_counters, epoch, wait,
                                      dev->stream);
    }
    start_gpu(dev);
    hipError_t e = clear_static_slots(dev, fixed, (extent + 3) / 4 * 4);
    if (e != hipSuccess) return e;
    wait.reset_slots = true;
    e = qmr::launch_dense_mfma(w, x, y, rows, cols, batch, pl, reinterpret_cast<unsigned long long *>(fixed),
                               reinterpret_cast<uint32_t *>(fixed + part), 1u, wait, dev->stream);
    if (e != hipSuccess) mark_static_dirty(dev, extent);
    return e;
}

// One packed-affine product of at most four RHS: the row-band matrix-core
// kernel where it has a plan whose workgroups are all resident at once; else
// the split-K matrix-core kernel where it supports the format, unless
// rows_preferred() hands the shape to the row-owning matrix-core kernel;
// else the vector-ALU kernels. A forced plan (testing hook) of rr > 0 or
// rr == -1 selects the vector-ALU tilings, rr == -4 the row-band kernel,
// rr == -3 the row-owning matrix-core kernel, rr == -2 the split-K kernel
// whatever its shape (with ks > 0 splits, when that count is feasible).
// `fixed` (qmr_encode_static) puts every workspace in the static scratch.
hipError_t launch_product(qmr_device *dev, const qmr::AffineArgs &a, unsigned char *fixed) {
    qmr::GemvPlan f = dev->forced_plan;
    if ((f.rr == 0 || f.rr == -4) && qmr::affine_tile_supported(a)) {
        const qmr::TilePlan pl = forced_tile_plan(dev, a, band_schedule(dev));
        if (pl.kw > 0) return launch_band(dev, a, pl, fixed);
    }
    if (f.rr == -4) f = qmr::GemvPlan{};  // no band plan for this shape: the default chain
    if (f.rr == -3 && qmr::affine_rows_supported(a)) {
        const qmr::RowsPlan pl = forced_rows_plan(dev, a);
        if (pl.rt > 0) {
            dev->last_hip = "affine_rows_kernel";
            start_gpu(dev);
            return qmr::launch_affine_rows(a, pl, dev->stream);
        }
    }
    if ((f.rr == 0 || f.rr == -2 || f.rr == -3) && qmr::affine_mfma_supported(a)) {
        const qmr::MfmaPlan pl =
            qmr::plan_affine_mfma(a, dev->limits, f.rr == -2 && f.ks > 0 ? uint32_t(f.ks) : 0u);
        if (f.rr == 0 && pl.rt > 0 && rows_preferred(pl) && qmr::affine_rows_supported(a)) {
            const qmr::RowsPlan rp = qmr::plan_affine_rows(a, dev->limits);
            if (rp.rt > 0) {
                dev->last_hip = "affine_rows_kernel";
                start_gpu(dev);
                return qmr::launch_affine_rows(a, rp, dev->stream);
            }
        }
        if (pl.rt > 0) {
            dev->last_hip = "affine_mfma_kernel";
            return launch_split_k(dev, a, pl, fixed);
        }
    }
    // The vector-ALU kernels have no fused epilogue.
    ensure(a.residual == nullptr, "fused product needs a matrix-core kernel", QMR_ERR_UNSUPPORTED);
    dev->last_hip = "affine_gemv_kernel";
    start_gpu(dev);
    return qmr::launch_affine_gemv(a, f.rr < -1 ? qmr::GemvPlan{} : f, dev->limits, dev->stream);
}

}  // namespace

extern "C" {

const char *qmr_last_error(void) { return g_error.c_str(); }

int qmr_device_open(int ordinal, const qmr_device_options *options, qmr_device **out) {
    return guarded([&]() -> int {
        ensure(out != nullptr, "qmr_device_open: null output");
        *out = nullptr;
        qmr_device_options opt{};
        if (options) opt = *options;
        std::string variant = opt.gemv_variant ? opt.gemv_variant : "aligned";
        ensure(is_variant(variant), "QWEN_METAL_GEMV must be packed4, aligned or stream");
        std::string metadata = opt.metadata_mode ? opt.metadata_mode : "f32";
        ensure(metadata == "f32" || metadata == "bf16", "QWEN_METAL_METADATA must be f32 or bf16");
        int count = 0;
        hipError_t e = hipGetDeviceCount(&count);
        ensure(e == hipSuccess && count > 0,
               "No HIP GPU available; this backend requires an AMD Instinct GPU (gfx950)",
               QMR_ERR_DEVICE);
        ensure(ordinal >= 0 && ordinal < count, "GPU ordinal out of range", QMR_ERR_INVALID);
        hipDeviceProp_t prop;
        check_hip(hipGetDeviceProperties(&prop, ordinal), "hipGetDeviceProperties");
        std::string arch = prop.gcnArchName;
        ensure(arch.rfind("gfx950", 0) == 0,
               "Kernels are built for gfx950 (MI355X); device reports " + arch, QMR_ERR_DEVICE);
        auto *dev = new qmr_device();
        dev->ordinal = ordinal;
        dev->name = prop.name[0] ? std::string(prop.name)
                                  : "AMD Instinct " + arch.substr(0, arch.find(':'));
        dev->gemv_variant = variant;
        dev->reference = opt.reference != 0;
        dev->bf16_metadata = metadata == "bf16" && !dev->reference;
        try {
            dev->block_mode =
                qmr::parse_block_kernel_mode_for_device(dev->name, opt.block_matmul, opt.block_delta);
        } catch (...) {
            delete dev;
            throw;
        }
        dev->max_alloc = prop.totalGlobalMem;
        dev->limits.max_lds_per_block = prop.sharedMemPerBlock;
        dev->limits.num_cus = prop.multiProcessorCount;
        e = hipSetDevice(ordinal);
        if (e == hipSuccess) e = hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            delete dev;
            check_hip(e, "hipStreamCreate");
        }
        try {
            const ScratchEntry se = scratch_entry(ordinal);
            dev->scratch = se.address;
            dev->scratch_dirty = se.dirty;
            void *st = nullptr;
            check_hip(hipHostMalloc(&st, 64, hipHostMallocMapped | hipHostMallocCoherent), "hipHostMalloc (status)");
            dev->status_host = static_cast<uint32_t *>(st);
            std::memset(st, 0, 64);
            void *sd = nullptr;
            check_hip(hipHostGetDevicePointer(&sd, st, 0), "hipHostGetDevicePointer (status)");
            dev->status_dev = static_cast<uint32_t *>(sd);
        } catch (...) {
            if (dev->status_host) hipHostFree(dev->status_host);
            hipStreamDestroy(dev->stream);
            delete dev;
            throw;
        }
        *out = dev;
        return QMR_OK;
    });
}

void qmr_device_close(qmr_device *device) {
    if (!device) return;
    hipSetDevice(device->ordinal);
    if (device->stream) {
        hipStreamSynchronize(device->stream);
        hipStreamDestroy(device->stream);
    }
    if (device->ws_wide) hipFree(device->ws_wide);
    if (device->ws_slots) hipFree(device->ws_slots);
    if (device->ws_counters) hipFree(device->ws_counters);
    if (device->status_host) hipHostFree(device->status_host);
    for (int i = 0; i < qmr::kStageSlots; ++i) {
        if (device->pin[i]) hipHostFree(device->pin[i]);
        if (device->pin_done[i]) hipEventDestroy(device->pin_done[i]);
    }
    delete device;
}

const char *qmr_device_name(const qmr_device *device) { return device ? device->name.c_str() : ""; }

const char *qmr_kernel_mode(const qmr_device *device) {
    if (!device) return "";
    return device->reference ? "reference" : device->gemv_variant.c_str();
}

const char *qmr_metadata_mode(const qmr_device *device) {
    return device && device->bf16_metadata ? "bf16" : "f32";
}

void qmr_block_kernel_mode(const qmr_device *device, int *matmul, int *batched_delta) {
    if (!device) return;
    if (matmul) *matmul = static_cast<int>(device->block_mode.matmul);
    if (batched_delta) *batched_delta = device->block_mode.batched_delta ? 1 : 0;
}

int qmr_set_block_kernel_mode(qmr_device *device, int matmul, int batched_delta) {
    return guarded([&]() -> int {
        ensure(device != nullptr, "null device");
        ensure(matmul >= 0 && matmul <= 2, "invalid block matmul mode");
        device->block_mode.matmul = static_cast<qmr::BlockMatmulMode>(matmul);
        device->block_mode.batched_delta = batched_delta != 0;
        return QMR_OK;
    });
}

int qmr_compact_metadata(const qmr_device *device, uint32_t bits, size_t group,
                         const float *scales, const float *biases, size_t n, uint16_t *s_out,
                         uint16_t *b_out) {
    if (!device || !device->bf16_metadata || !qmr::supported_bf16_quantization(bits, group))
        return 0;
    if (!qmr::pack_bf16_exact(scales, n, s_out)) return 0;
    if (!qmr::pack_bf16_exact(biases, n, b_out)) return 0;
    return 1;
}

void qmr_record_compacted_metadata(qmr_device *device, uint64_t saved_bytes) {
    if (!device) return;
    device->compacted_matrices += 1;
    device->metadata_saved_bytes += saved_bytes;
}

void qmr_metadata_stats(const qmr_device *device, size_t *matrices, uint64_t *saved_bytes) {
    if (!device) return;
    if (matrices) *matrices = device->compacted_matrices;
    if (saved_bytes) *saved_bytes = device->metadata_saved_bytes;
}

// ---- buffers ----

int qmr_buffer_alloc(qmr_device *device, size_t bytes, qmr_buffer **out) {
    return guarded([&]() -> int {
        ensure(device && out, "qmr_buffer_alloc: null argument");
        *out = nullptr;
        const size_t n = bytes < 4 ? 4 : bytes;
        ensure(n <= device->max_alloc, "GPU allocation " + std::to_string(n) +
                                           " exceeds device buffer limit " +
                                           std::to_string(device->max_alloc));
        check_hip(hipSetDevice(device->ordinal), "hipSetDevice");
        void *p = nullptr;
        check_hip(hipMalloc(&p, n), "hipMalloc");
        // Zeroed on the device stream and waited for, so the fill is ordered
        // before both later launches and host reads.
        hipError_t e = hipMemsetAsync(p, 0, n, device->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(device->stream);
        if (e != hipSuccess) {
            hipFree(p);
            check_hip(e, "hipMemsetAsync");
        }
        auto *b = new qmr_buffer();
        b->ordinal = device->ordinal;
        b->ptr = p;
        b->length = n;
        *out = b;
        return QMR_OK;
    });
}

int qmr_buffer_upload(qmr_device *device, const void *data, size_t bytes, qmr_buffer **out) {
    return guarded([&]() -> int {
        ensure(device && out, "qmr_buffer_upload: null argument");
        *out = nullptr;
        if (bytes == 0) return qmr_buffer_alloc(device, 0, out);
        ensure(data != nullptr, "qmr_buffer_upload: null data");
        ensure(bytes <= device->max_alloc, "GPU allocation " + std::to_string(bytes) +
                                               " exceeds device buffer limit " +
                                               std::to_string(device->max_alloc));
        check_hip(hipSetDevice(device->ordinal), "hipSetDevice");
        void *p = nullptr;
        check_hip(hipMalloc(&p, bytes), "hipMalloc");
        hipError_t e = hipMemcpy(p, data, bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            hipFree(p);
            check_hip(e, "hipMemcpy");
        }
        auto *b = new qmr_buffer();
        b->ordinal = device->ordinal;
        b->ptr = p;
        b->length = bytes;
        *out = b;
        return QMR_OK;
    });
}

int qmr_buffer_read(const qmr_buffer *buffer, size_t offset, void *dst, size_t bytes) {
    return guarded([&]() -> int {
        ensure(buffer && (dst || bytes == 0), "qmr_buffer_read: null argument");
        size_t end;
        ensure(!__builtin_add_overflow(offset, bytes, &end) && end <= buffer->length,
               "Read exceeds GPU buffer");
        if (bytes == 0) return QMR_OK;
        check_hip(hipSetDevice(buffer->ordinal), "hipSetDevice");
        check_hip(hipMemcpy(dst, static_cast<const char *>(buffer->ptr) + offset, bytes,
                            hipMemcpyDeviceToHost),
                  "hipMemcpy");
        return QMR_OK;
    });
}

int qmr_buffer_write(qmr_buffer *buffer, size_t offset, const void *src, size_t bytes) {
    return guarded([&]() -> int {
        ensure(buffer && (src || bytes == 0), "qmr_buffer_write: null argument");
        size_t end;
        ensure(!__builtin_add_overflow(offset, bytes, &end) && end <= buffer->length,
               "Write exceeds GPU buffer");
        if (bytes == 0) return QMR_OK;
        check_hip(hipSetDevice(buffer->ordinal), "hipSetDevice");
        check_hip(hipMemcpy(static_cast<char *>(buffer->ptr) + offset, src, bytes,
                            hipMemcpyHostToDevice),
                  "hipMemcpy");
        return QMR_OK;
    });
}

size_t qmr_buffer_length(const qmr_buffer *buffer) { return buffer ? buffer->length : 0; }

void qmr_buffer_retain(qmr_buffer *buffer) {
    if (buffer) buffer->refs.fetch_add(1);
}

void qmr_buffer_release(qmr_buffer *buffer) {
    if (!buffer) return;
    if (buffer->refs.fetch_sub(1) == 1) {
        hipSetDevice(buffer->ordinal);
        hipFree(buffer->ptr);
        delete buffer;
    }
}

// ---- commands ----

int qmr_command_begin(qmr_device *device, qmr_command **out) {
    return guarded([&]() -> int {
        ensure(device && out, "qmr_command_begin: null argument");
        *out = nullptr;
        check_hip(hipSetDevice(device->ordinal), "hipSetDevice");
        auto *cmd = new qmr_command();
        cmd->device = device;
        cmd->started = std::chrono::steady_clock::now();
        hipEvent_t ev;
        const hipError_t e = hipEventCreate(&ev);
        if (e != hipSuccess) {
            delete cmd;
            check_hip(e, "hipEventCreate");
        }
        cmd->marks.push_back(ev);
        // A command opened before this one that has launched nothing starts
        // here; this one starts at its first launch.
        if (device->pending) record_start(device->pending);
        device->pending = cmd;
        *out = cmd;
        return QMR_OK;
    });
}

int qmr_command_mark(qmr_command *command, int *index) {
    return guarded([&]() -> int {
        ensure(command && !command->finished, "qmr_command_mark: command not open");
        hipEvent_t ev;
        check_hip(hipEventCreate(&ev), "hipEventCreate");
        hipError_t e = hipEventRecord(ev, command->device->stream);
        if (e != hipSuccess) {
            hipEventDestroy(ev);
            check_hip(e, "hipEventRecord");
        }
        command->marks.push_back(ev);
        if (index) *index = int(command->marks.size()) - 1;
        return QMR_OK;
    });
}

int qmr_command_delay(qmr_command *command, uint32_t microseconds) {
    return guarded([&]() -> int {
        ensure(command && !command->finished, "qmr_command_delay: command not open");
        ensure(microseconds <= 1000000u, "qmr_command_delay: at most 1000000 microseconds");
        check_hip(hipSetDevice(command->device->ordinal), "hipSetDevice");
        int khz = 0;
        check_hip(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, command->device->ordinal),
                  "hipDeviceGetAttribute");
        ensure(khz > 0, "qmr_command_delay: the device reports no real-time clock rate", QMR_ERR_DEVICE);
        start_gpu(command->device);
        check_hip(qmr::launch_delay(uint64_t(microseconds) * uint64_t(khz) / 1000u, command->device->stream),
                  "delay launch");
        return QMR_OK;
    });
}

int qmr_command_finish(qmr_command *command, qmr_frame_timing *timing) {
    return guarded([&]() -> int {
        ensure(command && !command->finished, "qmr_command_finish: command not open");
        using clock = std::chrono::steady_clock;
        const double encode = std::chrono::duration<double>(clock::now() - command->started).count();
        const auto commit_start = clock::now();
        record_start(command);  // a command that launched nothing: zero GPU time
        hipEvent_t end;
        check_hip(hipEventCreate(&end), "hipEventCreate");
        hipError_t e = hipEventRecord(end, command->device->stream);
        if (e != hipSuccess) {
            hipEventDestroy(end);
            check_hip(e, "hipEventRecord");
        }
        command->marks.push_back(end);
        command->end_mark = int(command->marks.size()) - 1;
        const double commit = std::chrono::duration<double>(clock::now() - commit_start).count();
        const auto wait_start = clock::now();
        e = hipEventSynchronize(end);
        const double wait = std::chrono::duration<double>(clock::now() - wait_start).count();
        command->finished = true;
        if (e == hipSuccess) e = hipGetLastError();
        check_hip(e, "GPU command failed");
        // A launch of this command whose last K split gave up waiting for
        // the other splits' sums (row-band kernel: its band's workgroups were
        // not all resident at once; split-K kernel: a tagged slot never
        // arrived) wrote NaN for that band: the command failed, as a Metal
        // command buffer whose status is not Completed does
        // (src/gpu.rs:861-865). The static scratch may then hold sums that no
        // launch cleared.
        qmr_device *dev = command->device;
        const uint32_t status = __atomic_load_n(dev->status_host, __ATOMIC_ACQUIRE);
        if (status != 0) {
            __atomic_store_n(dev->status_host, 0u, __ATOMIC_RELEASE);
            mark_static_dirty(dev, QMR_STATIC_SCRATCH_BYTES);
            const bool band_kernel = (status & 0x60000000u) == 0;
            const char *kernel = (status & 0x40000000u) ? "affine_mfma_kernel"
                                 : (status & 0x20000000u) ? "dense_mfma_kernel"
                                                           : "affine_band_kernel";
            throw Error{QMR_ERR_DEVICE,
                        std::string("GPU command failed: ") + kernel + " band " +
                            std::to_string(status & 0x1FFFFFFFu) +
                            (band_kernel ? ": the last K split gave up waiting for the other splits' sums (the band's "
                                           "workgroups were not all resident at once)"
                                         : ": the last K split gave up waiting for the other splits' tagged sums") +
                            "; the command's outputs are not valid"};
        }
        float ms = 0.f;
        check_hip(hipEventElapsedTime(&ms, command->marks[0], end), "hipEventElapsedTime");
        if (timing) {
            timing->cpu_encode_seconds = encode;
            timing->cpu_commit_seconds = commit;
            timing->gpu_seconds = double(ms) * 1e-3;
            timing->completion_wait_seconds = wait;
        }
        return QMR_OK;
    });
}

int qmr_command_elapsed(const qmr_command *command, int from, int to, double *ms) {
    return guarded([&]() -> int {
        ensure(command && command->finished, "qmr_command_elapsed: command not finished");
        ensure(from >= 0 && to >= 0 && size_t(from) < command->marks.size() &&
                   size_t(to) < command->marks.size(),
               "qmr_command_elapsed: unknown mark");
        float v = 0.f;
        check_hip(hipEventElapsedTime(&v, command->marks[from], command->marks[to]),
                  "hipEventElapsedTime");
        if (ms) *ms = v;
        return QMR_OK;
    });
}

void qmr_command_release(qmr_command *command) {
    if (!command) return;
    if (command->device->pending == command) command->device->pending = nullptr;
    if (!command->finished) hipStreamSynchronize(command->device->stream);
    for (hipEvent_t ev : command->marks) hipEventDestroy(ev);
    delete command;
}

// ---- encode: the checked dispatch path of Gpu::encode_inner
// (src/gpu.rs:628-848): layout, buffer views, aliasing, mode bans,
// selection, thread and group checks, then the launch. ----

// The body of qmr_encode and qmr_encode_static; with no_alloc every launch
// takes its workspace from the static scratch and nothing is allocated.
static int encode_command(qmr_command *command, const char *cname, qmr_buffer *const *buffers,
                          const size_t *offsets, size_t nbuffers, const uint32_t *params, size_t nparams,
                          size_t threads, size_t group_size, bool no_alloc) {
    return guarded([&]() -> int {
        ensure(command && !command->finished, "qmr_encode: command not open");
        ensure(cname != nullptr, "qmr_encode: null kernel name");
        qmr_device *dev = command->device;
        unsigned char *fixed = no_alloc ? dev->scratch : nullptr;
        ensure(!no_alloc || fixed != nullptr, "qmr_encode_static: the device has no static scratch",
               QMR_ERR_DEVICE);
        const std::string name = cname;
        ensure(params != nullptr || nparams == 0, "qmr_encode: null params");
        const qmr::Layout layout = qmr::dispatch_layout(name, params, nparams);
        ensure(!dev->reference || !qmr::starts_with(name, "matmul_"),
               "Block matrix dispatch is unavailable in reference mode");
        ensure(layout.sizes.size() == nbuffers, name + ": expected " +
                                                    std::to_string(layout.sizes.size()) +
                                                    " buffers, got " + std::to_string(nbuffers));
        auto off = [&](size_t i) -> size_t { return offsets ? offsets[i] : 0; };
        for (size_t i = 0; i < nbuffers; ++i) {
            ensure(buffers[i] != nullptr, name + ": buffer " + std::to_string(i) + " is null");
            ensure(buffers[i]->ordinal == dev->ordinal,
                   name + ": buffer " + std::to_string(i) + " belongs to another device");
            try {
                qmr::checked_buffer_range(off(i), layout.sizes[i], buffers[i]->length);
            } catch (const Error &e) {
                throw Error{e.code, name + ": buffer " + std::to_string(i) + ": " + e.message};
            }
        }
        // A matrix-block output is never an input; a copy's views are
        // disjoint or identical (src/gpu.rs:658-672). The fused forms follow
        // the block rule, except that y may be exactly the residual's view
        // (the in-place x += W a of a decoder layer).
        const bool fused = qmr::is_fused_name(name);
        ensure(!dev->reference || !fused, "Fused dispatch is unavailable in reference mode");
        if (qmr::starts_with(name, "matmul_") || name == "copy_f32" || name == "read_checksum" || fused) {
            const size_t out = nbuffers - 1;
            for (size_t i = 0; i < out; ++i) {
                if (buffers[i] == buffers[out]) {
                    const bool identical_copy = (name == "copy_f32" || (qmr::is_residual_name(name) && i == 4)) &&
                                                off(i) == off(out);
                    ensure(identical_copy ||
                               !qmr::ranges_overlap(off(i), layout.sizes[i], off(out), layout.sizes[out]),
                           name + ": output overlaps input buffer " + std::to_string(i));
                }
            }
        }
        const qmr::Meta meta = qmr::meta_of_name(name);
        // src/gpu.rs:688-691.
        ensure(!dev->reference || !qmr::ends_with(name, "_bf16"),
               "BF16 metadata dispatch is unavailable in reference mode");
        ensure(!dev->reference || meta != qmr::Meta::F16,
               "F16 metadata dispatch is unavailable in reference mode");

        // Selection: the reference pipeline the Metal backend would pick
        // (src/gpu.rs:692-760). It decides the thread-group contract and is
        // recorded for inspection; the HIP instance is chosen below.
        const char *label = nullptr;
        const bool aligned_variant = dev->gemv_variant == "aligned";
        const bool wide = qmr::is_wide_name(name);
        if (qmr::starts_with(name, "matmul_") && !wide && !fused && meta != qmr::Meta::F16) {
            label = qmr::specialized_matmul(
                name, params,
                aligned_variant && off(0) % 8 == 0 && off(name == "matmul_f16" ? 1 : 3) % 16 == 0,
                dev->block_mode.matmul);
            ensure(label != nullptr, "Unsupported matrix block specialization", QMR_ERR_UNSUPPORTED);
        } else if (name == "matvec_affine_bf16") {
            ensure(off(3) % 16 == 0, "BF16 matvec input requires a 16-byte aligned offset");
            label = qmr::specialized_matvec_bf16(params, aligned_variant && off(0) % 8 == 0);
            ensure(label != nullptr, "Unsupported BF16 affine quantization", QMR_ERR_UNSUPPORTED);
        } else if (!dev->reference && name == "matvec_affine" && off(3) % 16 == 0) {
            if (dev->gemv_variant == "stream" && off(0) % 8 == 0 && params[2] == 4 &&
                uint64_t(params[0]) * params[1] <= uint64_t(INT32_MAX)) {
                if (params[3] == 32) label = "matvec_q4_g32_stream";
                if (params[3] == 64) label = "matvec_q4_g64_stream";
                if (params[3] == 128) label = "matvec_q4_g128_stream";
            }
            if (!label) label = qmr::specialized_matvec(params, aligned_variant && off(0) % 8 == 0);
        }
        ensure(threads == layout.threads, name + ": expected " + std::to_string(layout.threads) +
                                              " threads, got " + std::to_string(threads));
        const size_t actual_group =
            (label && (qmr::ends_with(label, "_aligned") || qmr::ends_with(label, "_aligned_bf16") ||
                       qmr::ends_with(label, "_stream")))
                ? 64
                : group_size;
        ensure(group_size >= 32 && group_size % 32 == 0 && actual_group <= pipeline_max_threads(label),
               name + ": invalid threadgroup size " + std::to_string(group_size));

        dev->last_kernel = label ? label : name;
        dev->last_hip = name;  // the families below name their own kernel
        check_hip(hipSetDevice(dev->ordinal), "hipSetDevice");
        auto ptr = [&](size_t i) -> char * {
            return static_cast<char *>(buffers[i]->ptr) + off(i);
        };
        hipError_t e = hipSuccess;
        // Families that launch without workspace start the frame's GPU time
        // here; the others start it after their workspace is in place.
        if (!qmr::starts_with(name, "mat") && !fused) start_gpu(dev);
        if (qmr::starts_with(name, "embed_affine")) {
            e = qmr::launch_embed_affine(reinterpret_cast<const uint32_t *>(ptr(0)), ptr(1), ptr(2),
                                         meta, params[0], params[1], params[2], params[3],
                                         reinterpret_cast<float *>(ptr(3)), dev->stream);
        } else if (name == "read_checksum") {
            e = qmr::launch_read_checksum(ptr(0), params[0], ptr(1), params[1], ptr(2), params[2],
                                          reinterpret_cast<uint32_t *>(ptr(3)), dev->read_plan, dev->stream);
        } else if (name == "copy_f32") {
            e = qmr::launch_copy_f32(reinterpret_cast<const float *>(ptr(0)),
                                     reinterpret_cast<float *>(ptr(1)), params[0], dev->limits.num_cus,
                                     dev->stream);
        } else if (name == "embed_f16") {
            e = qmr::launch_embed_f16(reinterpret_cast<const uint16_t *>(ptr(0)), params[0],
                                      params[1], reinterpret_cast<float *>(ptr(1)), dev->stream);
        } else if (name == "matvec_f16" || name == "matmul_f16") {
            const uint32_t batch = name == "matmul_f16" ? params[2] : 1;
            e = launch_dense(dev, reinterpret_cast<const uint16_t *>(ptr(0)), reinterpret_cast<const float *>(ptr(1)),
                             reinterpret_cast<float *>(ptr(2)), params[0], params[1], batch, fixed);
        } else if (fused) {
            qmr::AffineArgs a{};
            a.rows = params[0];
            a.cols = params[1];
            a.bits = params[2];
            a.group = params[3];
            a.batch = params[4];
            a.meta = meta;
            a.w = reinterpret_cast<const uint32_t *>(ptr(0));
            a.s = ptr(1);
            a.b = ptr(2);
            if (qmr::is_mlp_name(name)) {
                a.up_w = reinterpret_cast<const uint32_t *>(ptr(3));
                a.up_s = ptr(4);
                a.up_b = ptr(5);
                a.x = reinterpret_cast<const float *>(ptr(6));
                a.norm = reinterpret_cast<const float *>(ptr(7));
                a.y = reinterpret_cast<float *>(ptr(8));
                std::memcpy(&a.eps, &params[5], 4);
                ensure(qmr::affine_rows_supported(a), name + ": no fused kernel for this format",
                       QMR_ERR_UNSUPPORTED);
                // The row-band kernel's MLP form (bands of gate tiles and the
                // up tiles of the same rows) where it has a one-round plan (or
                // the tuning hook forces it, rr == -4); else the split-K
                // kernel (measured at 17408x5120:
                // 26.1 us at B=1 and 30.4 at B=3 against 29.4 and 35.5 for
                // the row-owning MLP mode, although both matrices' grid takes
                // two rounds of resident workgroups), also when the hook asks
                // for it (rr == -2, with ks > 0 K splits when feasible); the
                // row-owning kernel's MLP mode when
                // the hook asks for it (rr == -3, ks = j*10000 + rt*100 + kw)
                // or split-K has no plan.
                const qmr::GemvPlan f = dev->forced_plan;
                qmr::TilePlan bp;
                if ((f.rr == 0 || f.rr == -4) && qmr::affine_tile_supported(a)) bp = forced_tile_plan(dev, a);
                const qmr::MfmaPlan mp =
                    bp.kw > 0 ? qmr::MfmaPlan{}
                              : qmr::plan_affine_mfma(a, dev->limits, f.rr == -2 && f.ks > 0 ? uint32_t(f.ks) : 0u);
                if (bp.kw > 0) {
                    e = launch_band(dev, a, bp, fixed);
                    dev->last_hip += " (MLP)";
                } else if (f.rr != -3 && mp.rt > 0) {
                    dev->last_hip = "affine_mfma_kernel (MLP)";
                    e = launch_split_k(dev, a, mp, fixed);
                } else {
                    const qmr::RowsPlan pl =
                        f.rr == -3 && f.ks > 0
                            ? qmr::plan_affine_mlp(a, dev->limits, uint32_t(f.ks / 100 % 100), uint32_t(f.ks % 100),
                                                   uint32_t(f.ks / 10000))
                            : qmr::plan_affine_mlp(a, dev->limits);
                    ensure(pl.rt > 0, name + ": no fused tiling for this shape", QMR_ERR_UNSUPPORTED);
                    dev->last_hip = "affine_rows_kernel (MLP)";
                    start_gpu(dev);
                    e = qmr::launch_affine_rows(a, pl, dev->stream);
                }
            } else {
                a.x = reinterpret_cast<const float *>(ptr(3));
                a.residual = reinterpret_cast<const float *>(ptr(4));
                a.y = reinterpret_cast<float *>(ptr(5));
                ensure(qmr::affine_mfma_supported(a), name + ": no fused kernel for this format",
                       QMR_ERR_UNSUPPORTED);
                e = launch_product(dev, a, fixed);
            }
        } else {
            qmr::AffineArgs a{};
            a.w = reinterpret_cast<const uint32_t *>(ptr(0));
            a.s = ptr(1);
            a.b = ptr(2);
            a.x = reinterpret_cast<const float *>(ptr(3));
            a.y = reinterpret_cast<float *>(ptr(4));
            a.rows = params[0];
            a.cols = params[1];
            a.bits = params[2];
            a.group = params[3];
            a.batch = qmr::starts_with(name, "matmul_") ? params[4] : 1;
            a.meta = meta;
            const bool fast_group = a.group == 32 || a.group == 64 || a.group == 128;
            // The wide kernel takes RHS in blocks of 32 and measures about
            // 33 us at 17408x5120 for any batch up to 32, against 15.8 us for
            // one split-K block of four: batches of up to eight run as blocks.
            if (wide && qmr::wide_mfma_supported(a) && a.batch > 8) {
                const size_t need = qmr::wide_mfma_workspace(a);
                unsigned char *images = fixed;
                if (fixed) {
                    check_static_scratch(need, "wide-block activation images");
                    mark_static_dirty(dev, need);
                }
                if (!fixed && need > dev->ws_wide_bytes) {
                    check_hip(hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
                    if (dev->ws_wide) hipFree(dev->ws_wide);
                    dev->ws_wide = nullptr;
                    dev->ws_wide_bytes = 0;
                    check_hip(hipMalloc(&dev->ws_wide, need), "hipMalloc (wide workspace)");
                    dev->ws_wide_bytes = need;
                }
                if (!fixed) images = dev->ws_wide;
                dev->last_hip = "wide_mfma_kernel";
                start_gpu(dev);
                e = qmr::launch_wide_mfma(a, images, dev->limits, dev->stream);
            } else if (wide) {
                // Wide blocks of up to eight RHS, and those outside the wide
                // kernel's format, run as successive blocks of up to four RHS.
                for (uint32_t t0 = 0; t0 < a.batch && e == hipSuccess; t0 += 4) {
                    qmr::AffineArgs sub = a;
                    sub.batch = a.batch - t0 < 4 ? a.batch - t0 : 4;
                    sub.x = a.x + size_t(t0) * a.cols;
                    sub.y = a.y + size_t(t0) * a.rows;
                    e = launch_product(dev, sub, fixed);
                }
            } else if (dev->reference || !fast_group) {
                dev->last_hip = "affine_generic_kernel";
                start_gpu(dev);
                e = qmr::launch_affine_generic(a, dev->stream);
            } else {
                e = launch_product(dev, a, fixed);
            }
        }
        check_hip(e, "kernel launch");
        return QMR_OK;
    });
}

int qmr_wide_address_extent(uint32_t rows, uint32_t cols, uint32_t batch, uint32_t row_tiles, uint64_t *out) {
    return guarded([&]() -> int {
        ensure(out != nullptr, "qmr_wide_address_extent: null output");
        ensure(rows > 0 && cols > 0 && cols % 256 == 0 && batch >= 1 && batch <= 256 &&
                   (row_tiles == 8 || row_tiles == 17) && uint64_t(rows) * cols / 2 < (1ull << 31),
               "qmr_wide_address_extent: unsupported shape");
        const qmr::WideExtent e = qmr::wide_address_extent(rows, cols, batch, row_tiles);
        out[0] = e.code_end;
        out[1] = e.code_extent;
        out[2] = e.image_end;
        out[3] = e.image_extent;
        return QMR_OK;
    });
}

int qmr_encode(qmr_command *command, const char *name, qmr_buffer *const *buffers,
               const size_t *offsets, size_t nbuffers, const uint32_t *params, size_t nparams,
               size_t threads, size_t group_size) {
    return encode_command(command, name, buffers, offsets, nbuffers, params, nparams, threads, group_size,
                          false);
}

int qmr_encode_static(qmr_command *command, const char *name, qmr_buffer *const *buffers,
                      const size_t *offsets, size_t nbuffers, const uint32_t *params, size_t nparams,
                      size_t threads, size_t group_size) {
    return encode_command(command, name, buffers, offsets, nbuffers, params, nparams, threads, group_size,
                          true);
}

// ---- host-only contract functions ----

int qmr_dispatch_layout(const char *name, const uint32_t *params, size_t nparams, size_t *sizes,
                        size_t max_sizes, size_t *nsizes, size_t *threads) {
    return guarded([&]() -> int {
        ensure(name != nullptr, "null kernel name");
        const qmr::Layout l = qmr::dispatch_layout(name, params, nparams);
        ensure(l.sizes.size() <= max_sizes, "size array too small");
        for (size_t i = 0; i < l.sizes.size(); ++i) sizes[i] = l.sizes[i];
        if (nsizes) *nsizes = l.sizes.size();
        if (threads) *threads = l.threads;
        return QMR_OK;
    });
}

int qmr_checked_buffer_range(size_t offset, size_t minimum, size_t length) {
    return guarded([&]() -> int {
        qmr::checked_buffer_range(offset, minimum, length);
        return QMR_OK;
    });
}

int qmr_ranges_overlap(size_t a, size_t a_len, size_t b, size_t b_len) {
    return qmr::ranges_overlap(a, a_len, b, b_len) ? 1 : 0;
}

const char *qmr_specialized_matvec(const uint32_t *params, int aligned, int bf16) {
    return bf16 ? qmr::specialized_matvec_bf16(params, aligned != 0)
                : qmr::specialized_matvec(params, aligned != 0);
}

const char *qmr_specialized_matmul(const char *name, const uint32_t *params, size_t nparams,
                                   int aligned, int mode) {
    if (!name || !params) return nullptr;
    const std::string n = name;
    if ((n == "matmul_f16" && nparams != 3) || (n != "matmul_f16" && nparams != 5)) return nullptr;
    return qmr::specialized_matmul(n, params, aligned != 0, static_cast<qmr::BlockMatmulMode>(mode));
}

int qmr_parse_block_kernel_mode(const char *device_name, const char *matmul, const char *delta,
                                int *matmul_out, int *batched_delta_out) {
    return guarded([&]() -> int {
        const qmr::BlockKernelMode m = qmr::parse_block_kernel_mode_for_device(
            device_name ? device_name : "", matmul, delta);
        if (matmul_out) *matmul_out = static_cast<int>(m.matmul);
        if (batched_delta_out) *batched_delta_out = m.batched_delta ? 1 : 0;
        return QMR_OK;
    });
}

int qmr_pack_bf16_exact(const float *values, size_t n, uint16_t *out) {
    return qmr::pack_bf16_exact(values, n, out) ? 1 : 0;
}

int qmr_supported_bf16_quantization(uint32_t bits, size_t group) {
    return qmr::supported_bf16_quantization(bits, group) ? 1 : 0;
}

// ---- testing / tuning hooks (declared in include/qmr_tuning.h) ----

int qmr_set_read_plan(qmr_device *device, uint32_t workgroups, uint32_t unroll, int nontemporal) {
    return guarded([&]() -> int {
        ensure(device != nullptr, "null device");
        ensure(workgroups <= qmr::kChecksumSlots, "read_checksum: at most 4096 workgroups");
        ensure(unroll == 0 || unroll == 1 || unroll == 2 || unroll == 4 || unroll == 8,
               "read_checksum: loads in flight per thread must be 1, 2, 4 or 8 (0 = default)");
        ensure(nontemporal >= -1 && nontemporal <= 1, "read_checksum: nontemporal must be -1, 0 or 1");
        device->read_plan.workgroups = workgroups;
        device->read_plan.unroll = unroll;
        device->read_plan.nt = nontemporal;
        return QMR_OK;
    });
}

int qmr_set_band_wait_fault(qmr_device *device, int enabled) {
    return guarded([&]() -> int {
        ensure(device != nullptr, "null device");
        device->force_give_up = enabled != 0;
        return QMR_OK;
    });
}

int qmr_set_gemv_plan(qmr_device *device, int rr, int ks) {
    return guarded([&]() -> int {
        ensure(device != nullptr, "null device");
        device->forced_plan.rr = rr;
        device->forced_plan.ks = ks;
        return QMR_OK;
    });
}

const char *qmr_last_kernel(const qmr_device *device) {
    return device ? device->last_kernel.c_str() : "";
}

const char *qmr_last_hip_kernel(const qmr_device *device) {
    return device ? device->last_hip.c_str() : "";
}

int qmr_gemv_plan(const qmr_device *device, uint32_t rows, uint32_t cols, uint32_t bits,
                  uint32_t batch, int *rr, int *ks) {
    return guarded([&]() -> int {
        ensure(device != nullptr, "null device");
        if (bits == 16) {
            // Dense F16 (an aligned view): rr = -5, ks = ring*10000 +
            // kw*1000 + rt*100 + ns on the matrix-core kernel, else rr = -1
            // (vector-ALU kernels).
            const qmr::DensePlan pl =
                dense_plan(device, reinterpret_cast<const uint16_t *>(uintptr_t(256)), rows, cols, batch);
            if (rr) *rr = pl.rt > 0 ? -5 : -1;
            if (ks) *ks = pl.rt > 0 ? int(pl.ring * 10000 + pl.kw * 1000 + pl.rt * 100 + pl.ns) : 0;
            return QMR_OK;
        }
        qmr::AffineArgs a{};
        a.rows = rows;
        a.cols = cols;
        a.bits = bits;
        a.group = 64;
        a.batch = batch;
        a.meta = qmr::Meta::BF16;
        qmr::GemvPlan f = device->forced_plan;
        if ((f.rr == 0 || f.rr == -4) && qmr::affine_tile_supported(a)) {
            const qmr::TilePlan pl = forced_tile_plan(device, a);
            if (pl.kw > 0) {
                // Row-band kernel: rr = -4, ks = ring*100000 + ns*10000 + tr*100 + kw.
                if (rr) *rr = -4;
                if (ks) *ks = int((pl.phases == 2 ? 2000000 : 0) + pl.ring * 100000 + pl.ns * 10000 + pl.tr * 100 + pl.kw);
                return QMR_OK;
            }
        }
        if (f.rr == -4) f = qmr::GemvPlan{};
        if (f.rr == -3 && qmr::affine_rows_supported(a)) {
            const qmr::RowsPlan pl = forced_rows_plan(device, a);
            if (pl.rt > 0) {
                // Row-owning kernel: rr = -3, ks = j*10000 + rt*100 + kw.
                if (rr) *rr = -3;
                if (ks) *ks = int(pl.j * 10000 + pl.rt * 100 + pl.kw);
                return QMR_OK;
            }
        }
        if ((f.rr == 0 || f.rr == -2 || f.rr == -3) && qmr::affine_mfma_supported(a)) {
            const qmr::MfmaPlan pl =
                qmr::plan_affine_mfma(a, device->limits, f.rr == -2 && f.ks > 0 ? uint32_t(f.ks) : 0u);
            if (f.rr == 0 && pl.rt > 0 && rows_preferred(pl) && qmr::affine_rows_supported(a)) {
                const qmr::RowsPlan rp = qmr::plan_affine_rows(a, device->limits);
                if (rp.rt > 0) {
                    if (rr) *rr = -3;
                    if (ks) *ks = int(rp.j * 10000 + rp.rt * 100 + rp.kw);
                    return QMR_OK;
                }
            }
            if (pl.rt > 0) {
                // Matrix-core kernel: rr = -2, ks = K splits across workgroups.
                if (rr) *rr = -2;
                if (ks) *ks = int(pl.ns);
                return QMR_OK;
            }
        }
        const qmr::GemvPlan p = qmr::plan_affine_gemv(a, f.rr < -1 ? qmr::GemvPlan{} : f,
                                                      device->limits);
        if (rr) *rr = p.rr;
        if (ks) *ks = p.ks;
        return QMR_OK;
    });
}

size_t qmr_device_workspace_bytes(const qmr_device *device) {
    if (!device) return 0;
    return device->ws_slots_bytes + device->ws_counter_count * sizeof(uint32_t) +
           device->ws_wide_bytes;
}

size_t qmr_device_max_lds(const qmr_device *device) {
    return device ? device->limits.max_lds_per_block : 0;
}

}  // extern "C"

#!/usr/bin/env python3
"""Benchmark of the packed-affine GEMV hot path on one MI355X.

Metric: Q4/g64 GEMV time and achieved HBM GB/s (fraction of
the 8 TB/s peak) at 5120x17408 (the MLP down projection, rows x K) at B=1 and
B=3; the 17408x5120 gate/up shape moves the same bytes and is reported too.

A step is one launch of the metric kernel over one synthetic input batch
(Q4/g64 codes, BF16 scales/biases, FP32 x), all resident in HBM before the
timed region starts. Weights rotate over --copies distinct copies so that the
50 MB matrix is not served from the 256 MB Infinity Cache.

Timing: K launches run back to back between two HIP events recorded on the
library's stream; their difference over K is the mean launch duration, and
`value` is the algorithmic bytes of one launch (codes + scales + biases + x +
y) divided by it. Ahead of the start event a one-wave kernel holds the stream
for 40 us per launch (qmr_command_delay), so that all K launches are queued
before the GPU reaches them and the events time the GPU, not the host's
enqueue rate. The wall time of the timed region (synchronised on both sides)
less that hold gives ms_per_step. A second pass brackets each launch with its own
events to report the spread. Before the W warmup launches of each case, about
1 s of untimed launches lets the GPU clocks settle after the host-side idle
of building that case's matrix.

The CPU baseline times the FP64 oracle (the reference's per-weight
dequantise-then-accumulate closure, restated in C) on this host.

The read floor: read_checksum streams the metric matrix's codes, scales and
biases (the same rotating copies, the same timing) and does nothing else, in
three read geometries; the fastest is reported as roofline.read_floor_us and
roofline.frac_of_floor is that time over the GEMV's. --floor-sweep sweeps it
over sizes and geometries instead of running the bench.

BASELINE config 3 (the Q8/g64 F16 5120x5120 projection, the same matrix with
FP32 metadata, and the Q4/g64 BF16 151936x5120 vocabulary head, B=1 and B=3)
is reported under "config3" with an HBM roofline per case.

One decoder layer's MLP in the fused forms (RMS norm + gate + up + SwiGLU in
one launch, down + residual add in a second) is reported under "mlp", beside
the three plain products timed alone.

Dense F16 products (matvec_f16 / matmul_f16) at the MLP shapes are reported
under "dense_f16".

The checkpoint loader (MLX safetensors to device buffers) is timed on one
layer's three MLP matrices and reported under "loader" (host-to-device GB/s).

The reference's shared-weight block microbenchmark (B GEMVs in one command
against one block dispatch, alternating AB/BA, medians of the frame GPU
time) runs at the metric shape with B=3 and is reported under
"block_vs_sequential".

BASELINE config 4 (the wide block: 17408x5120 Q4/g64 BF16 times 128 and 256
FP32 columns) is timed the same way and reported under "wide" with its own
matrix-core roofline (algorithmic FLOP against the dense f16 peak); it is not
the headline metric.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "qwen-mlx-runner_amd"))

import numpy as np  # noqa: E402

import qmr  # noqa: E402
import qmr.synth as synth  # noqa: E402

METRIC = "Q4/g64 GEMV µs + achieved HBM GB/s (% peak), 5120x17408 at B=1 and B=3"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16 matrix-core peak


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


SETTLE_MS = 1000.0
HOLD_US = 40  # GPU-side hold per timed launch, ahead of the start mark


def settle(gpu: qmr.Gpu, name: str, bufsets, params, threads: int, ms: float, static: bool = False) -> None:
    """Untimed launches until about `ms` of GPU time has run. The clocks ramp
    up over a few hundred milliseconds of load after the host has kept the
    GPU idle (as it does while it builds each synthetic matrix): on MI355X
    the first timed region of the 5120x17408 GEMV read 14.8 us after 50 ms of
    such launches, 14.1 us after 200 ms and a steady 13.8 us after 1 s; the
    vocabulary head read 90 us cold against 77 us steady."""
    cmd = gpu.begin()
    a = cmd.mark()
    for k in range(10):
        cmd.encode(name, bufsets[k % len(bufsets)], params, threads, 128, static_scratch=static)
    b = cmd.mark()
    cmd.finish()
    per = max(cmd.elapsed_ms(a, b) / 10, 1e-3)
    cmd.release()
    cmd = gpu.begin()
    for k in range(int(ms / per)):
        cmd.encode(name, bufsets[k % len(bufsets)], params, threads, 128, static_scratch=static)
    cmd.finish()
    cmd.release()


def time_kernel(gpu: qmr.Gpu, name: str, bufsets, params, steps: int, warmup: int, static: bool = False):
    """Back-to-back launch timing (events at both ends of the timed region),
    plus per-launch event brackets for the spread. Returns
    (mean ms per launch back-to-back, wall seconds of that region,
     per-launch bracketed durations in ms). `static` encodes through
    qmr_encode_static (workspace in the static scratch)."""
    _, threads = qmr.dispatch_layout(name, params)
    settle(gpu, name, bufsets, params, threads, SETTLE_MS, static)
    enc = lambda cmd, k: cmd.encode(name, bufsets[k % len(bufsets)], params, threads, 128, static_scratch=static)
    cmd = gpu.begin()
    for k in range(warmup):
        enc(cmd, k)
    cmd.finish()
    cmd.release()
    # Timed region: synchronised on both sides, K launches back to back. A
    # GPU-side hold ahead of the start mark (HOLD_US per launch) keeps the
    # GPU from reaching the launches before the host has queued them all, so
    # the marks time the GPU and not the host's enqueue rate (7-14 us per
    # launch through this Python binding, which is slower than a 12 us GEMV
    # on some hosts).
    cmd = gpu.begin()
    hold_us = min(HOLD_US * steps, 1_000_000)
    cmd.delay(hold_us)
    t0 = time.perf_counter()
    a = cmd.mark()
    for k in range(steps):
        enc(cmd, k)
    b = cmd.mark()
    enqueue_us = (time.perf_counter() - t0) * 1e6
    cmd.finish()
    # Wall time of the region less the hold, which the GPU starts as the host
    # starts enqueueing: the K launches plus the synchronisation.
    wall = time.perf_counter() - t0 - hold_us * 1e-6
    mean_ms = cmd.elapsed_ms(a, b) / steps
    cmd.release()
    if enqueue_us > hold_us:
        log(f"bench:   warning: enqueueing {steps} launches took {enqueue_us:.0f} us, longer than the "
            f"{hold_us} us hold; the timing may include host gaps")
    # Spread: each launch bracketed by its own pair of events (adds the
    # event overhead to every sample, so these read a little high).
    cmd = gpu.begin()
    marks = []
    n = min(steps, 100)
    cmd.delay(min(HOLD_US * 3 * n, 1_000_000))
    for k in range(n):
        a = cmd.mark()
        enc(cmd, k)
        marks.append((a, cmd.mark()))
    cmd.finish()
    durs = [cmd.elapsed_ms(a, b) for a, b in marks]
    cmd.release()
    return mean_ms, wall, durs


def cpu_baseline(m: synth.PackedMatrix, budget_s: float) -> dict:
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    threads = max(1, min(cores, 16))
    x = synth.activations(m.cols, 1, synth.DEFAULT_SEED, tag="bench")
    run = lambda th, f: f(m.w, m.s, m.b, m.meta, x, m.rows, m.cols, m.bits, m.group, 1, th)
    t = time.perf_counter()
    run(threads, oracle.matmul_f64)
    first = time.perf_counter() - t
    reps = int(max(2, min(20, budget_s * 0.6 / max(first, 1e-3))))
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        run(threads, oracle.matmul_f64)
        times.append(time.perf_counter() - t)
    t = time.perf_counter()
    run(1, oracle.matmul_f64)
    single = time.perf_counter() - t
    t = time.perf_counter()
    run(threads, oracle.matmul_f32)
    f32 = time.perf_counter() - t
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    med = statistics.median(times)
    nbytes = synth.algorithmic_bytes(m, 1)
    return {
        "value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"FP64 oracle (oracle/qmr_oracle.c, per-weight dequantise then FP64 "
                   f"accumulate) on the full {m.rows}x{m.cols} Q4/g64 BF16 B=1 matrix "
                   f"({nbytes} algorithmic bytes), median of {reps} runs on {threads} threads"),
        "us_per_matrix": round(med * 1e6, 1),
        "single_thread_us": round(single * 1e6, 1),
        "fp32_accumulate_us": round(f32 * 1e6, 1),
        "cpu_model": model, "host_cores_visible": cores,
    }


def copy_calibration(gpu: qmr.Gpu, mib: int, launches: int) -> None:
    """Plain copies of a known size (copy_f32: `mib` MiB read and `mib` MiB
    written per launch, over two buffer pairs) for calibrating rocprofv3's
    FETCH_SIZE / WRITE_SIZE counters in the same process as the metric
    kernel. Not part of the timed metric."""
    n = mib * (1 << 20) // 4
    pairs = [(gpu.upload_f32(np.ones(n, np.float32)), gpu.alloc_f32(n)) for _ in range(2)]
    cmd = gpu.begin()
    for k in range(launches):
        src, dst = pairs[k % 2]
        cmd.encode("copy_f32", [src, dst], [n], n, 128)
    cmd.finish()
    cmd.release()
    log(f"bench: copy calibration, {launches} x copy_f32 of {mib} MiB")
    del pairs


def bench_wide(gpu: qmr.Gpu, args) -> list:
    """the 17408x5120 Q4/g64 BF16 matrix times 128 and 256
    FP32 columns (matmul_affine_wide_bf16), 4 rotating weight copies."""
    rows, cols = synth.MLP_SHAPES["gate_up"]
    m = synth.q4_bf16_matrix(rows, cols, synth.DEFAULT_SEED, tag="gate_up")
    mats = [(gpu.upload_bytes(m.w), gpu.upload_bytes(m.s), gpu.upload_bytes(m.b)) for _ in range(4)]
    out = []
    for batch in (128, 256):
        x = synth.activations(cols, batch, synth.DEFAULT_SEED, tag="wide")
        xb = gpu.upload_f32(x.ravel())
        ys = [gpu.alloc_f32(batch * rows) for _ in range(len(mats))]
        bufsets = [[w, s, b, xb, y] for (w, s, b), y in zip(mats, ys)]
        log(f"bench: wide {rows}x{cols} x {batch} (matmul_affine_wide_bf16)")
        mean_ms, _, _ = time_kernel(gpu, "matmul_affine_wide_bf16", bufsets, [rows, cols, 4, 64, batch],
                                    args.wide_steps, 5)
        flop = 2.0 * rows * cols * batch
        tflops = flop / (mean_ms * 1e-3) / 1e12
        r = {
            "shape": f"{rows}x{cols}", "rhs": batch, "us_mean": round(mean_ms * 1e3, 2),
            "roofline": {
                "bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                "note": "algorithmic FLOP (2*rows*cols*rhs); the kernel issues twice that on the "
                        "matrix cores (x split into hi/lo f16 parts)",
            },
        }
        log(f"bench:   {r['us_mean']} us, {r['roofline']['achieved']} TFLOP/s algorithmic = "
            f"{100 * r['roofline']['frac']:.1f}% of the f16 MFMA peak")
        out.append(r)
        del bufsets, ys, xb
    del mats
    return out


def bench_config3(gpu: qmr.Gpu, args) -> list:
    """the Q8/g64 F16-metadata 5120x5120 attention
    projection and the Q4/g64 BF16 151936x5120 vocabulary head, each at B=1
    and B=3. Weights rotate over enough copies to exceed the Infinity Cache
    (10 of the 26 MB projection, 2 of the 440 MB head)."""
    q8 = synth.q8_f16_matrix(5120, 5120, synth.DEFAULT_SEED, tag="q8")
    cases = [("q8_proj", q8, 10), ("q8_proj_f32meta", synth.to_f32_metadata(q8), 10),
             ("head", synth.q4_bf16_matrix(*synth.HEAD_SHAPE, synth.DEFAULT_SEED, tag="head"), 2)]
    out = []
    for tag, m, copies in cases:
        mats = [(gpu.upload_bytes(m.w), gpu.upload_bytes(m.s), gpu.upload_bytes(m.b))
                for _ in range(copies)]
        suffix = {"f16": "_f16meta", "bf16": "_bf16", "f32": ""}[m.meta]
        for batch in (1, 3):
            x = synth.activations(m.cols, batch, synth.DEFAULT_SEED, tag="bench")
            xb = gpu.upload_f32(x.ravel())
            ys = [gpu.alloc_f32(batch * m.rows) for _ in range(copies)]
            bufsets = [[w, s, b, xb, y] for (w, s, b), y in zip(mats, ys)]
            name = ("matvec_affine" if batch == 1 else "matmul_affine") + suffix
            params = [m.rows, m.cols, m.bits, m.group] + ([batch] if batch > 1 else [])
            log(f"bench: {tag} {m.rows}x{m.cols} Q{m.bits} B={batch} ({name})")
            mean_ms, _, _ = time_kernel(gpu, name, bufsets, params, args.config3_steps, 6)
            nbytes = synth.algorithmic_bytes(m, batch)
            gbps = nbytes / (mean_ms * 1e-3) / 1e9
            plan = gpu.gemv_plan(m.rows, m.cols, m.bits, batch)
            r = {
                "shape": f"{m.rows}x{m.cols}", "tag": tag, "bits": m.bits, "metadata": m.meta,
                "batch": batch, "kernel": hip_kernel(plan), "hip_launch": gpu.last_hip_kernel(),
                "plan": list(plan),
                "us_mean": round(mean_ms * 1e3, 2), "algorithmic_bytes": nbytes,
                "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBS,
                             "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBS, 4)},
            }
            log(f"bench:   {r['us_mean']} us, {r['roofline']['achieved']} GB/s = "
                f"{100 * r['roofline']['frac']:.1f}% of peak ({r['kernel']})")
            out.append(r)
            del bufsets, ys, xb
        floor = read_floor(gpu, m, mats, args, steps=args.config3_steps)
        log(f"bench:   {tag} read floor {floor['us_mean']} us ({floor['gbps']} GB/s)")
        for r in out:
            if r["tag"] == tag:
                r["read_floor_us"] = floor["us_mean"]
                r["frac_of_floor"] = round(floor["us_mean"] / r["us_mean"], 4)
        del mats
    return out


def bench_mlp(gpu: qmr.Gpu, args) -> list:
    """One decoder layer's MLP with the fused forms: mlp_gate_up_swiglu_bf16
    (RMS norm, gate and up 17408x5120, SwiGLU: one launch) then
    matmul_affine_add_bf16 (down 5120x17408 plus the residual add, in place),
    at B=1 and B=3. The reference runs the same layer as seven launches
    (src/engine.rs:748-765); beside the fused pair this times the three
    plain products alone (matvec/matmul_affine_bf16), which the unfused
    sequence needs on top of its four elementwise launches."""
    ku, kd = synth.MLP_SHAPES["gate_up"], synth.MLP_SHAPES["down"]
    copies = 4
    mats = {}
    for tag, (rows, cols) in (("gate", ku), ("up", ku), ("down", kd)):
        m = synth.q4_bf16_matrix(rows, cols, synth.DEFAULT_SEED, tag=tag)
        mats[tag] = [(gpu.upload_bytes(m.w), gpu.upload_bytes(m.s), gpu.upload_bytes(m.b)) for _ in range(copies)]
        nbytes_w = m.w.nbytes + m.s.nbytes + m.b.nbytes
    eps_bits = int(np.float32(1e-6).view(np.uint32))
    hidden, inter = ku[1], ku[0]
    norm = gpu.upload_f32(np.random.default_rng(1).uniform(0.5, 1.5, hidden).astype(np.float32))
    out = []
    for batch in (1, 3):
        x = gpu.upload_f32(synth.activations(hidden, batch, synth.DEFAULT_SEED, tag="mlp").ravel())
        act = gpu.alloc_f32(batch * inter)
        resid = gpu.upload_f32(np.zeros(batch * hidden, np.float32))
        up_sets = [[*mats["gate"][k], *mats["up"][k], x, norm, act] for k in range(copies)]
        dn_sets = [[*mats["down"][k], act, resid, resid] for k in range(copies)]
        up_params = [inter, hidden, 4, 64, batch, eps_bits]
        dn_params = [hidden, inter, 4, 64, batch]
        _, up_threads = qmr.dispatch_layout("mlp_gate_up_swiglu_bf16", up_params)
        _, dn_threads = qmr.dispatch_layout("matmul_affine_add_bf16", dn_params)
        settle(gpu, "mlp_gate_up_swiglu_bf16", up_sets, up_params, up_threads, SETTLE_MS)
        cmd = gpu.begin()
        for k in range(5):
            cmd.encode("mlp_gate_up_swiglu_bf16", up_sets[k % copies], up_params, up_threads, 128)
            cmd.encode("matmul_affine_add_bf16", dn_sets[k % copies], dn_params, dn_threads, 128)
        cmd.finish()
        cmd.release()
        cmd = gpu.begin()
        cmd.delay(min(2 * HOLD_US * args.mlp_steps, 1_000_000))
        a = cmd.mark()
        for k in range(args.mlp_steps):
            cmd.encode("mlp_gate_up_swiglu_bf16", up_sets[k % copies], up_params, up_threads, 128)
            cmd.encode("matmul_affine_add_bf16", dn_sets[k % copies], dn_params, dn_threads, 128)
        b = cmd.mark()
        cmd.finish()
        layer_ms = cmd.elapsed_ms(a, b) / args.mlp_steps
        cmd.release()
        # The three plain products alone, back to back, for comparison.
        name = "matvec_affine_bf16" if batch == 1 else "matmul_affine_bf16"
        extra = [] if batch == 1 else [batch]
        xi = gpu.upload_f32(np.zeros(batch * inter, np.float32))
        yg, yu, yd = gpu.alloc_f32(batch * inter), gpu.alloc_f32(batch * inter), gpu.alloc_f32(batch * hidden)
        seq = []
        for k in range(copies):
            seq.append((name, [*mats["gate"][k], x, yg], [inter, hidden, 4, 64] + extra))
            seq.append((name, [*mats["up"][k], x, yu], [inter, hidden, 4, 64] + extra))
            seq.append((name, [*mats["down"][k], xi, yd], [hidden, inter, 4, 64] + extra))
        thr = [qmr.dispatch_layout(n, p_)[1] for n, _, p_ in seq]
        cmd = gpu.begin()
        cmd.delay(min(3 * HOLD_US * args.mlp_steps, 1_000_000))
        a = cmd.mark()
        for k in range(args.mlp_steps):
            for j in range(3):
                n, bufs, p_ = seq[(3 * k + j) % len(seq)]
                cmd.encode(n, bufs, p_, thr[(3 * k + j) % len(seq)], 128)
        b = cmd.mark()
        cmd.finish()
        plain_ms = cmd.elapsed_ms(a, b) / args.mlp_steps
        cmd.release()
        nbytes = 3 * nbytes_w + 4 * batch * (hidden + inter + inter + hidden + hidden) + 4 * hidden
        gbps = nbytes / (layer_ms * 1e-3) / 1e9
        r = {"workload": "decoder MLP, 27B shapes, Q4/g64 BF16", "batch": batch, "launches": 2,
             "us_layer": round(layer_ms * 1e3, 2), "us_three_plain_products": round(plain_ms * 1e3, 2),
             "algorithmic_bytes": nbytes,
             "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(gbps / HBM_PEAK_GBS, 4)}}
        log(f"bench: fused MLP B={batch}: {r['us_layer']} us per layer in 2 launches "
            f"({r['roofline']['achieved']} GB/s, {100 * r['roofline']['frac']:.1f}% of peak); "
            f"the 3 plain products alone {r['us_three_plain_products']} us")
        out.append(r)
    del mats
    return out


def bench_dense(gpu: qmr.Gpu, args) -> list:
    """Dense F16 products at the 27B MLP shapes (matvec_f16 / matmul_f16,
    kernels/qwen.metal:48-57, kernels/matmul_block.metal:213-248), for
    checkpoints without quantisation: 178 MB of F16 weights, 3 rotating
    copies, B=1 and B=3, with the kernel the default choice ran; at B=3 the
    vector-ALU kernel is timed beside it (the rr = -1 hook)."""
    out = []
    for tag in ("down", "gate_up"):
        rows, cols = synth.MLP_SHAPES[tag]
        w16 = np.random.default_rng(7).standard_normal(rows * cols).astype(np.float16).view(np.uint16)
        ws = [gpu.upload_bytes(w16) for _ in range(3)]
        del w16
        for batch in (1, 3):
            xb = gpu.upload_f32(synth.activations(cols, batch, synth.DEFAULT_SEED, tag="dense").ravel())
            ys = [gpu.alloc_f32(batch * rows) for _ in ws]
            name = "matvec_f16" if batch == 1 else "matmul_f16"
            params = [rows, cols] + ([batch] if batch > 1 else [])
            bufs = [[w, xb, y] for w, y in zip(ws, ys)]
            mean_ms, _, _ = time_kernel(gpu, name, bufs, params, args.config3_steps, 6)
            kernel = gpu.last_hip_kernel()
            nbytes = rows * cols * 2 + 4 * batch * (rows + cols)
            gbps = nbytes / (mean_ms * 1e-3) / 1e9
            r = {"shape": f"{rows}x{cols}", "batch": batch, "name": name, "kernel": kernel,
                 "us_mean": round(mean_ms * 1e3, 2), "algorithmic_bytes": nbytes,
                 "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(gbps / HBM_PEAK_GBS, 4)}}
            if batch > 1:
                gpu.set_gemv_plan(-1, 0)
                try:
                    valu_ms, _, _ = time_kernel(gpu, name, bufs, params, args.config3_steps, 6)
                finally:
                    gpu.set_gemv_plan(0, 0)
                r["us_vector_alu"] = round(valu_ms * 1e3, 2)
            log(f"bench: dense F16 {rows}x{cols} B={batch} ({kernel}): {r['us_mean']} us, "
                f"{r['roofline']['achieved']} GB/s = {100 * r['roofline']['frac']:.1f}% of peak"
                + (f"; vector-ALU kernel {r['us_vector_alu']} us" if batch > 1 else ""))
            out.append(r)
        del ws
    return out


PCIE_PEAK_GBS = 64.0  # PCIe 5.0 x16, one direction


def bench_loader(args) -> dict:
    """The checkpoint loader: one layer's three MLP matrices (gate and up
    17408x5120, down 5120x17408, Q4/g64 with BF16 metadata) written as an MLX
    safetensors checkpoint in a temporary directory, then opened and loaded
    into a "bf16" device (qmr_checkpoint_open + qmr_matrix_load, the
    reference's Checkpoint::open + Matrix::load). The file is in the page
    cache, as after a first load; the figure is host-to-device throughput."""
    import shutil
    import struct
    import tempfile

    def write_tensor_file(path: Path, tensors) -> None:
        # safetensors: 8-byte header length, JSON header, data section.
        header, data = {}, []
        pos = 0
        for name, dtype, shape, payload in tensors:
            header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [pos, pos + len(payload)]}
            data.append(payload)
            pos += len(payload)
        h = json.dumps(header).encode()
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", len(h)) + h)
            for payload in data:
                f.write(payload)

    def write_config(d: Path, **extra) -> None:
        (d / "config.json").write_text(json.dumps({"model_type": "qwen3_5_text", **extra}))

    d = Path(tempfile.mkdtemp(prefix="qmr_ck_"))
    try:
        tensors, shapes = [], {}
        for proj, key in (("gate_proj", "gate_up"), ("up_proj", "gate_up"), ("down_proj", "down")):
            rows, cols = synth.MLP_SHAPES[key]
            m = synth.q4_bf16_matrix(rows, cols, synth.DEFAULT_SEED, tag=proj)
            name = f"language_model.model.layers.0.mlp.{proj}"
            tensors += [(name + ".weight", "U32", [rows, cols // 8], m.w.tobytes()),
                        (name + ".scales", "BF16", [rows, cols // 64], m.s.tobytes()),
                        (name + ".biases", "BF16", [rows, cols // 64], m.b.tobytes())]
            shapes[f"model.layers.0.mlp.{proj}"] = (rows, cols)
        write_config(d, quantization={"bits": 4, "group_size": 64, "mode": "affine"})
        write_tensor_file(d / "model.safetensors", tensors)
        del tensors
        nbytes = (d / "model.safetensors").stat().st_size
        gpu = qmr.Gpu("aligned", metadata="bf16")
        times = []
        for _ in range(args.loader_reps):
            t = time.perf_counter()
            with qmr.Checkpoint(d) as cp:
                loaded = [cp.load(gpu, n, r, c) for n, (r, c) in shapes.items()]
            times.append(time.perf_counter() - t)
            assert all(m.metadata_bf16 for m in loaded)
            del loaded
        gpu.close()
    finally:
        shutil.rmtree(d, ignore_errors=True)
    med = statistics.median(times)
    gbps = nbytes / med / 1e9
    r = {"workload": "3 MLP matrices (2 x 17408x5120 + 5120x17408, Q4/g64 BF16) from one safetensors file",
         "file_bytes": nbytes, "reps": len(times), "ms_median": round(med * 1e3, 2),
         "ms_min": round(min(times) * 1e3, 2),
         "roofline": {"bound": "pcie", "achieved": round(gbps, 2), "peak": PCIE_PEAK_GBS, "unit": "GB/s",
                      "frac": round(gbps / PCIE_PEAK_GBS, 4)}}
    log(f"bench: loader {nbytes / 1e6:.1f} MB in {r['ms_median']} ms = {gbps:.2f} GB/s")
    return r


def hip_kernel(plan) -> str:
    """The HIP kernel family the planner picked (plan[0]: -4 row-band matrix
    cores, -2 split-K matrix cores, -3 row-owning matrix cores, otherwise the
    vector-ALU kernel)."""
    return {-4: "affine_band_kernel", -2: "affine_mfma_kernel",
            -3: "affine_rows_kernel"}.get(plan[0], "affine_gemv_kernel")


def bench_block_vs_sequential(gpu: qmr.Gpu, iterations: int) -> dict:
    """The reference's shared-weight block microbenchmark
    (examples/block_matrix_bench.rs:28-172) at the metric shape with B=3: one
    command holding B separate GEMVs (matvec_affine_bf16 at x/y offsets of
    token t) against one command holding the block (matmul_affine_bf16),
    same weights, inputs and output buffer, five warmups per mode, then
    `iterations` of each in alternating AB/BA order; medians of the
    command's FrameTiming GPU time and of its wall time. The data is the
    reference benchmark's synthetic pattern. The two results must agree
    within the reference's bound (1e-3 + 5e-5*|y|). One weight copy, as in
    the reference: its 50 MB may be served from the Infinity Cache."""
    rows, cols, batch = 5120, 17408, 3
    total = rows * cols
    i = np.arange(total // 8, dtype=np.uint64)
    w = ((i * 0x9E3779B9 + 0x1478ABCF) & 0xFFFFFFFF).astype(np.uint32)
    g = np.arange(total // 64)
    scales = ((1 + g % 11) / 512.0).astype(np.float32)
    biases = ((g % 9) / 256.0 - 0.0625).astype(np.float32)
    inputs = ((np.arange(batch * cols) * 13 % 101 - 50) / 50.0).astype(np.float32)
    bf16 = lambda v: (v.view(np.uint32) >> 16).astype(np.uint16)
    bufs = [gpu.upload_bytes(w), gpu.upload_bytes(bf16(scales)), gpu.upload_bytes(bf16(biases)),
            gpu.upload_f32(inputs), gpu.alloc_f32(batch * rows)]
    log(f"bench: block vs sequential, {rows}x{cols} B={batch} ({iterations} per mode, AB/BA)")

    def measure(block: bool):
        t0 = time.perf_counter()
        cmd = gpu.begin()
        if block:
            cmd.encode("matmul_affine_bf16", bufs, [rows, cols, 4, 64, batch], rows * 32, 128)
        else:
            for t in range(batch):
                cmd.encode("matvec_affine_bf16", bufs, [rows, cols, 4, 64], rows * 32, 128,
                           offsets=[0, 0, 0, t * cols * 4, t * rows * 4])
        timing = cmd.finish()
        cmd.release()
        return timing.gpu_seconds, time.perf_counter() - t0

    for _ in range(5):
        measure(False)
        measure(True)
    times = {False: ([], []), True: ([], [])}
    for it in range(iterations):
        for block in (it % 2 == 0, it % 2 != 0):
            g_s, w_s = measure(block)
            times[block][0].append(g_s)
            times[block][1].append(w_s)
    measure(False)
    expected = gpu.read_f32(bufs[4], batch * rows)
    measure(True)
    actual = gpu.read_f32(bufs[4], batch * rows)
    diff = np.abs(actual.astype(np.float64) - expected)
    ok = bool(np.isfinite(actual).all() and (diff <= 1e-3 + np.abs(expected) * 5e-5).all())
    med = lambda v: float(statistics.median(v))
    r = {
        "kind": "shared_weight_matrix_block_microbenchmark",
        "rows": rows, "cols": cols, "batch": batch, "bits": 4, "group_size": 64, "metadata_mode": "bf16",
        "iterations_per_mode": iterations,
        "sequential_gpu_median_ms": round(med(times[False][0]) * 1e3, 4),
        "block_gpu_median_ms": round(med(times[True][0]) * 1e3, 4),
        "gpu_speedup": round(med(times[False][0]) / med(times[True][0]), 3),
        "sequential_wall_median_ms": round(med(times[False][1]) * 1e3, 4),
        "block_wall_median_ms": round(med(times[True][1]) * 1e3, 4),
        "max_absolute_difference": float(diff.max()),
        "within_reference_bound": ok,
    }
    log(f"bench:   sequential {r['sequential_gpu_median_ms']} ms, block {r['block_gpu_median_ms']} ms GPU "
        f"(speedup {r['gpu_speedup']}), max |diff| {r['max_absolute_difference']:.3g}")
    if not ok:
        raise AssertionError("block/GEMV mismatch beyond 1e-3 + 5e-5*|y|")
    return r


# Published results of the reference's kernel-bench on Apple M5 Pro
# (docs/benchmarks/m5-pro-aligned-kernels-user.json), FP32 metadata.
KERNEL_BENCH_PUBLISHED = {(17408, 5120): {"device": "Apple M5 Pro", "iterations": 100,
                                          "milliseconds_per_matvec": 0.24718958,
                                          "effective_weight_gb_per_second": 225.35577753722467},
                          (248320, 5120): {"device": "Apple M5 Pro", "iterations": 12,
                                           "milliseconds_per_matvec": 2.9875903333333333,
                                           "effective_weight_gb_per_second": 265.97488656131014}}


def kernel_bench(gpu: qmr.Gpu, rows: int, cols: int, iterations: int, bf16: bool, bits: int = 4,
                 group: int = 64) -> dict:
    """The reference's `kernel-bench` command (src/main.rs:552-644), same
    method: every packed word 0x76543210, every scale 0.015625 and bias
    -0.0625 (exact in BF16, so both metadata modes hold the same values),
    x = 0.1; one weight copy; 3 warmup dispatches in one command, then
    `iterations` dispatches of matvec_affine[_bf16] in one command, timed by
    the host wall clock from the command's begin to its finish;
    milliseconds_per_matvec and effective_weight_gb_per_second over the
    code, scale and bias bytes. The same weights are read every time, so on
    this device the matrix may be served from the 256 MB Infinity Cache (the
    reference's own note says so for its cache); the rotating-copy metric
    above is the one that excludes it."""
    elements = rows * cols
    w = np.full(elements // (32 // bits), 0x76543210, np.uint32)
    sv = np.full(elements // group, 0.015625, np.float32)
    bv = np.full(elements // group, -0.0625, np.float32)
    if bf16:
        sv, bv = synth.f32_to_bf16_bits(sv), synth.f32_to_bf16_bits(bv)
    bufs = [gpu.upload_bytes(w), gpu.upload_bytes(sv), gpu.upload_bytes(bv),
            gpu.upload_f32(np.full(cols, 0.1, np.float32)), gpu.alloc_f32(rows)]
    name = "matvec_affine_bf16" if bf16 else "matvec_affine"
    params = [rows, cols, bits, group]

    def dispatch(count: int) -> float:
        start = time.perf_counter()
        cmd = gpu.begin()
        for _ in range(count):
            cmd.encode(name, bufs, params, rows * 32, 128)
        cmd.finish()
        cmd.release()
        return time.perf_counter() - start

    dispatch(3)
    seconds = dispatch(iterations)
    y = gpu.read_f32(bufs[4], rows)
    if not np.isfinite(y).all():
        raise RuntimeError("kernel-bench: non-finite kernel output")
    # Every row is the same affine dot: sum over columns of (q*s + b)*0.1 with
    # q cycling 0..7 (the word 0x76543210).
    q = np.tile(np.arange(8, dtype=np.float64), cols // 8)
    want = float(((q * 0.015625 - 0.0625) * np.float64(np.float32(0.1))).sum())
    if not np.allclose(y, want, rtol=1e-5, atol=1e-5):
        raise RuntimeError(f"kernel-bench: output {y[:4]} differs from {want}")
    wbytes = sum(b.nbytes for b in (w, sv, bv))
    r = {"kind": "packed_matvec_microbenchmark", "bits": bits, "group_size": group,
         "kernel_mode": gpu.kernel_mode(), "metadata_mode": "bf16" if bf16 else "f32",
         "synthetic_metadata_values": {"scale": 0.015625, "bias": -0.0625},
         "device": gpu.name(), "rows": rows, "cols": cols, "iterations": iterations, "seconds": seconds,
         "milliseconds_per_matvec": seconds * 1000.0 / iterations,
         "effective_weight_gb_per_second": wbytes * iterations / seconds / 1e9,
         "hip_launch": gpu.last_hip_kernel(),
         "note": ("Repeated synthetic weights may benefit from cache (here the 256 MB Infinity Cache). "
                  "This is NOT model tokens per second."),
         "timing": "host wall clock from command begin to finish, as the reference's kernel-bench"}
    pub = KERNEL_BENCH_PUBLISHED.get((rows, cols))
    if pub and not bf16:
        r["reference_published"] = pub
    log(f"bench:   kernel-bench {rows}x{cols} {r['metadata_mode']} x{iterations}: "
        f"{r['milliseconds_per_matvec'] * 1e3:.2f} us per matvec, "
        f"{r['effective_weight_gb_per_second']:.1f} GB/s effective")
    for b in bufs:
        b.release()
    return r


def bench_kernel_bench(gpu: qmr.Gpu) -> list:
    """kernel_bench at the reference's default shape (17408x5120, 50
    iterations; its published run used 100), the metric's transpose and the
    reference's large published shape, in both metadata modes."""
    out = []
    for rows, cols, iters in ((17408, 5120, 100), (5120, 17408, 100), (248320, 5120, 12)):
        for bf16 in (False, True):
            log(f"bench: kernel-bench {rows}x{cols} {'bf16' if bf16 else 'f32'} metadata, {iters} iterations")
            out.append(kernel_bench(gpu, rows, cols, iters, bf16))
    return out


def bench_static_entry(gpu: qmr.Gpu, m: synth.PackedMatrix, mats, args) -> list:
    """The metric GEMV and block through qmr_encode_static (every workspace
    in the static scratch, nothing allocated) beside qmr_encode, timed the
    same way: the row-band split sums then need no fill launch between
    consecutive calls (the last splits clear the slots they take)."""
    out = []
    for batch in (1, 3):
        x = synth.activations(m.cols, batch, synth.DEFAULT_SEED, tag="bench")
        xb = gpu.upload_f32(x.ravel())
        ys = [gpu.alloc_f32(batch * m.rows) for _ in mats]
        bufsets = [[w, s, b, xb, y] for (w, s, b), y in zip(mats, ys)]
        name = "matvec_affine_bf16" if batch == 1 else "matmul_affine_bf16"
        params = [m.rows, m.cols, 4, 64] + ([batch] if batch > 1 else [])
        log(f"bench: qmr_encode_static {m.rows}x{m.cols} B={batch}")
        mean_ms, _, _ = time_kernel(gpu, name, bufsets, params, args.steps, args.warmup, static=True)
        out.append({"shape": f"{m.rows}x{m.cols}", "batch": batch, "entry": "qmr_encode_static",
                    "hip_launch": gpu.last_hip_kernel(), "us_mean": round(mean_ms * 1e3, 3),
                    "gbps": round(synth.algorithmic_bytes(m, batch) / (mean_ms * 1e-3) / 1e9, 1)})
        log(f"bench:   {out[-1]['us_mean']} us ({out[-1]['hip_launch']})")
        del bufsets, ys, xb
    return out


def floor_sweep(gpu: qmr.Gpu, args) -> dict:
    """read_checksum, the read floor, over sizes (25-500 MB, default
    geometry) and over its geometry at the metric matrix's 50.1 MB
    (workgroups, 16-byte loads in flight per thread, non-temporal or plain
    loads). Each size splits into three views in the metric matrix's
    proportions (codes, scales, biases); each case rotates over enough copies
    to exceed the 256 MB Infinity Cache (at least 10, and at least 1 GB),
    timed as the GEMV is."""
    m = synth.q4_bf16_matrix(*synth.MLP_SHAPES["down"], synth.DEFAULT_SEED, tag="down")
    frac = [m.w.nbytes / m.nbytes, m.s.nbytes / m.nbytes, m.b.nbytes / m.nbytes]
    outs = [gpu.alloc_f32(qmr.CHECKSUM_SLOTS) for _ in range(2)]

    def views(total: int, copies: int):
        sizes = [int(total * f) // 16 * 16 for f in frac]
        mats = [tuple(gpu.alloc_f32(n // 4) for n in sizes) for _ in range(copies)]
        return sizes, mats

    def run(sizes, mats, steps):
        bufsets = [[a, b, c, outs[k % 2]] for k, (a, b, c) in enumerate(mats)]
        mean_ms, _, durs = time_kernel(gpu, "read_checksum", bufsets, sizes, steps, 10)
        return mean_ms, durs

    res = {"sizes": [], "geometry": []}
    for mb in (25, 50, 100, 200, 500):
        total = m.nbytes * mb // 50
        copies = max(10, -(-(1 << 30) // total))
        sizes, mats = views(total, copies)
        log(f"bench: floor sweep, {sum(sizes)} bytes, {copies} copies, default geometry")
        mean_ms, durs = run(sizes, mats, max(40, min(args.steps, int(2e5 / mb))))
        res["sizes"].append({"bytes": sum(sizes), "copies": copies, "us_mean": round(mean_ms * 1e3, 3),
                             "us_p10_p50_p90": [round(v * 1e3, 3) for v in np.quantile(durs, [0.1, 0.5, 0.9])],
                             "gbps": round(sum(sizes) / (mean_ms * 1e-3) / 1e9, 1)})
        log(f"bench:   {res['sizes'][-1]['us_mean']} us, {res['sizes'][-1]['gbps']} GB/s")
        for t in mats:
            for b in t:
                b.release()
    sizes = [m.w.nbytes, m.s.nbytes, m.b.nbytes]
    mats = [tuple(gpu.alloc_f32(n // 4) for n in sizes) for _ in range(10)]
    for wg in (256, 512, 1024, 2048, 4080):
        for unroll in (1, 2, 4, 8):
            for nt in (1, 0):
                if nt == 0 and unroll not in (4, 8):
                    continue
                gpu.set_read_plan(wg, unroll, nt)
                mean_ms, durs = run(sizes, mats, args.steps)
                res["geometry"].append({"workgroups": wg, "loads_in_flight_per_thread": unroll,
                                        "kb_per_workgroup": round(sum(sizes) / wg / 1024, 1),
                                        "nontemporal": bool(nt), "us_mean": round(mean_ms * 1e3, 3),
                                        "gbps": round(sum(sizes) / (mean_ms * 1e-3) / 1e9, 1)})
                log(f"bench:   floor geometry wg={wg} unroll={unroll} nt={nt}: {res['geometry'][-1]['us_mean']} us")
    gpu.set_read_plan(0, 0, -1)
    mean_ms, _ = run(sizes, mats, args.steps)
    res["default_at_metric"] = {"bytes": sum(sizes), "us_mean": round(mean_ms * 1e3, 3)}
    return res


# read_checksum geometries (workgroups, 16-byte loads in flight per thread,
# non-temporal) the floor takes the fastest of: the three fastest of the
# geometry sweep at the metric matrix's 50 MB (profiles/read_checksum_floor_sweep.md),
# whose order changes from box to box.
FLOOR_GEOMETRIES = ((4080, 4, 1), (2048, 8, 1), (1024, 4, 1))


def read_floor(gpu: qmr.Gpu, m: synth.PackedMatrix, mats, args, steps: int = 0) -> dict:
    """The streaming-read floor of the metric launch: read_checksum (16-byte
    non-temporal loads over contiguous per-workgroup slices, XOR-reduced into
    4096 slots) reads the same codes, scales and biases over the same
    rotating copies, timed the same way as the GEMV, in each of
    FLOOR_GEOMETRIES; the floor is the fastest. It does no arithmetic beyond
    the XOR, so its time bounds what any kernel that reads these bytes once
    can take on this device; the XOR of the slots is checked against the
    host's XOR of every word."""
    outs = [gpu.alloc_f32(qmr.CHECKSUM_SLOTS) for _ in mats]
    bufsets = [[w, s, b, o] for (w, s, b), o in zip(mats, outs)]
    params = [m.w.nbytes, m.s.nbytes, m.b.nbytes]
    want = np.uint32(0)
    for a in (m.w, m.s, m.b):
        want ^= np.bitwise_xor.reduce(np.ascontiguousarray(a).view(np.uint32))
    runs = []
    for wg, unroll, nt in FLOOR_GEOMETRIES:
        gpu.set_read_plan(wg, unroll, nt)
        log(f"bench: read floor, read_checksum of {m.nbytes} bytes ({len(mats)} rotating copies), "
            f"{wg} workgroups x {unroll} loads in flight")
        mean_ms, _, durs = time_kernel(gpu, "read_checksum", bufsets, params, steps or args.steps, args.warmup)
        got = np.bitwise_xor.reduce(gpu.read_f32(outs[0], qmr.CHECKSUM_SLOTS).view(np.uint32))
        if got != want:
            raise RuntimeError(f"read_checksum XOR {got:#x} != host {want:#x}")
        runs.append({"workgroups": wg, "loads_in_flight_per_thread": unroll, "nontemporal": bool(nt),
                     "us_mean": round(mean_ms * 1e3, 3),
                     "us_bracketed_p10_p50_p90": [round(v * 1e3, 3) for v in np.quantile(durs, [0.1, 0.5, 0.9])]})
        log(f"bench:   {runs[-1]['us_mean']} us")
    gpu.set_read_plan(0, 0, -1)
    best = min(runs, key=lambda r: r["us_mean"])
    return {"kernel": "read_checksum_kernel", "bytes": int(m.nbytes), "us_mean": best["us_mean"],
            "geometry": {k: best[k] for k in ("workgroups", "loads_in_flight_per_thread", "nontemporal")},
            "us_bracketed_p10_p50_p90": best["us_bracketed_p10_p50_p90"],
            "gbps": round(m.nbytes / (best["us_mean"] * 1e-6) / 1e9, 1), "geometries": runs}


def load_traffic(tag: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by its copy_f32 calibration)."""
    p = ROOT / "profiles" / "pmc_traffic.json"
    if not p.exists():
        return None
    try:
        d = json.loads(p.read_text())
        return d.get(tag, {}).get("hbm_bytes_per_launch")
    except (ValueError, OSError):
        return None


def main() -> int:
    global SETTLE_MS
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only-metric", action="store_true",
                    help="time only the 5120x17408 shapes (for profiling runs)")
    ap.add_argument("--only-wide", action="store_true",
                    help="time only the config-4 wide block (for profiling runs)")
    ap.add_argument("--only-dense", action="store_true",
                    help="only time the dense F16 products (for profiling), print that JSON and exit")
    ap.add_argument("--wide-steps", type=int, default=30)
    ap.add_argument("--config3-steps", type=int, default=60)
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="untimed launches before each case, in ms of GPU time (clock ramp)")
    ap.add_argument("--loader-reps", type=int, default=5)
    ap.add_argument("--mlp-steps", type=int, default=100)
    ap.add_argument("--no-mlp", action="store_true", help="skip the fused decoder-MLP timing")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense F16 timing")
    ap.add_argument("--no-loader", action="store_true", help="skip the checkpoint-loader timing")
    ap.add_argument("--block-iters", type=int, default=100,
                    help="iterations per mode of the block vs sequential comparison (0 skips it)")
    ap.add_argument("--no-config3", action="store_true",
                    help="skip the config-3 Q8 projection and vocabulary head")
    ap.add_argument("--gemv-plan", default=None, metavar="RR,KS",
                    help="force the GEMV kernel and tiling (qmr_set_gemv_plan) for the metric shapes, "
                         "e.g. -1,0 for the vector-ALU kernel (profiling runs)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first run plain copies of MIB MiB (counter calibration for profiling)")
    ap.add_argument("--no-kernel-bench", action="store_true",
                    help="skip the reference's kernel-bench method (cache-warm host wall clock)")
    ap.add_argument("--floor-sweep", action="store_true",
                    help="only sweep read_checksum over sizes and geometries, print that JSON and exit")
    args = ap.parse_args()
    SETTLE_MS = args.settle_ms
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the hot path is "
              f"single-GPU; multi-GPU sharding is design-only)", file=sys.stderr)
        return 2
    if int(os.environ.get("RANK", "0")) != 0:
        return 0

    gpu = qmr.Gpu("aligned")
    log(f"bench: device {gpu.name()}, steps={args.steps} warmup={args.warmup} copies={args.copies}")
    if args.gemv_plan:
        rr, ks = (int(v) for v in args.gemv_plan.split(","))
        gpu.set_gemv_plan(rr, ks)
        log(f"bench: forced GEMV plan ({rr}, {ks})")
    if args.copy_calibration:
        copy_calibration(gpu, args.copy_calibration, 8)
    if args.floor_sweep:
        print(json.dumps({"floor_sweep": floor_sweep(gpu, args)}), flush=True)
        gpu.close()
        return 0
    if args.only_dense:
        print(json.dumps({"dense_f16": bench_dense(gpu, args)}), flush=True)
        gpu.close()
        return 0
    shapes = [] if args.only_wide else [("down", synth.MLP_SHAPES["down"])]
    if not args.only_metric and not args.only_wide:
        shapes.append(("gate_up", synth.MLP_SHAPES["gate_up"]))
    results = []
    metric_matrix = None
    floor = None
    static_entry = []
    for tag, (rows, cols) in shapes:
        m = synth.q4_bf16_matrix(rows, cols, synth.DEFAULT_SEED, tag=tag)
        if tag == "down":
            metric_matrix = m
        mats = [(gpu.upload_bytes(m.w), gpu.upload_bytes(m.s), gpu.upload_bytes(m.b))
                for _ in range(args.copies)]
        for batch in (1, 3):
            x = synth.activations(cols, batch, synth.DEFAULT_SEED, tag="bench")
            xb = gpu.upload_f32(x.ravel())
            ys = [gpu.alloc_f32(batch * rows) for _ in range(args.copies)]
            bufsets = [[w, s, b, xb, y] for (w, s, b), y in zip(mats, ys)]
            name = "matvec_affine_bf16" if batch == 1 else "matmul_affine_bf16"
            params = [rows, cols, 4, 64] + ([batch] if batch > 1 else [])
            log(f"bench: {tag} {rows}x{cols} B={batch} ({name})")
            mean_ms, wall, durs = time_kernel(gpu, name, bufsets, params, args.steps, args.warmup)
            nbytes = synth.algorithmic_bytes(m, batch)
            q = np.quantile(durs, [0.1, 0.5, 0.9])
            r = {
                "shape": f"{rows}x{cols}", "tag": tag, "batch": batch,
                "reference_pipeline": gpu.last_kernel(),
                "kernel": hip_kernel(gpu.gemv_plan(rows, cols, 4, batch)),
                "hip_launch": gpu.last_hip_kernel(),
                "plan": list(gpu.gemv_plan(rows, cols, 4, batch)),
                "us_mean": round(mean_ms * 1e3, 3),
                "us_bracketed_p10_p50_p90": [round(v * 1e3, 3) for v in q],
                "algorithmic_bytes": nbytes,
                "gbps": round(nbytes / (mean_ms * 1e-3) / 1e9, 1),
                "frac_peak": round(nbytes / (mean_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "wall_ms_per_step": round(wall / args.steps * 1e3, 4),
            }
            log(f"bench:   {r['us_mean']} us per launch back-to-back (bracketed p50 "
                f"{r['us_bracketed_p10_p50_p90'][1]}), {r['gbps']} GB/s = "
                f"{100 * r['frac_peak']:.1f}% of peak")
            results.append(r)
            del bufsets, ys, xb
        if tag == "down":
            floor = read_floor(gpu, m, mats, args)
            log(f"bench:   read floor {floor['us_mean']} us ({floor['gbps']} GB/s)")
            if not args.only_metric and not args.gemv_plan:
                static_entry = bench_static_entry(gpu, m, mats, args)
        del mats

    if args.gemv_plan:
        gpu.set_gemv_plan(0, 0)
    wide = [] if args.only_metric else bench_wide(gpu, args)
    if args.only_wide:
        print(json.dumps({"wide": wide}), flush=True)
        gpu.close()
        return 0
    config3 = [] if (args.only_metric or args.no_config3) else bench_config3(gpu, args)
    mlp = [] if (args.only_metric or args.no_mlp) else bench_mlp(gpu, args)
    dense = [] if (args.only_metric or args.no_dense) else bench_dense(gpu, args)
    loader = None if (args.only_metric or args.no_loader) else bench_loader(args)
    block_seq = None if (args.only_metric or args.block_iters <= 0) else bench_block_vs_sequential(gpu, args.block_iters)
    kbench = [] if (args.only_metric or args.no_kernel_bench) else bench_kernel_bench(gpu)
    head = next(r for r in results if r["tag"] == "down" and r["batch"] == 1)
    b3 = next(r for r in results if r["tag"] == "down" and r["batch"] == 3)
    cpu = None
    if not args.no_cpu and metric_matrix is not None:
        log("bench: CPU baseline (FP64 oracle)")
        cpu = cpu_baseline(metric_matrix, args.cpu_seconds)
        log(f"bench:   CPU {cpu['us_per_matrix']} us/matrix ({cpu['value']} GB/s) on "
            f"{cpu['cores']} threads")
    line = {
        "metric": METRIC,
        "value": head["gbps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms_per_case": SETTLE_MS,
        "ms_per_step": head["wall_ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": "Q4/g64 BF16-metadata GEMV 5120x17408 (rows x K), B=1; B=3 block alongside",
            "rows": 5120, "cols": 17408, "bits": 4, "group": 64, "metadata": "bf16",
            "batch": 1, "rotating_weight_copies": args.copies,
        },
        "us_b1": head["us_mean"], "gbps_b1": head["gbps"], "frac_b1": head["frac_peak"],
        "us_b3": b3["us_mean"], "gbps_b3": b3["gbps"], "frac_b3": b3["frac_peak"],
        "roofline": {
            "bound": "hbm",
            "achieved": head["gbps"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": head["frac_peak"],
            "traffic": load_traffic("down_b1"),
            "kernel": hip_kernel(head["plan"]),
            "launch": head["hip_launch"],
            # The same 50 MB read by read_checksum with the same rotation and
            # timing; frac_of_floor = floor time / GEMV time.
            "read_floor_us": floor["us_mean"] if floor else None,
            "read_floor_gbps": floor["gbps"] if floor else None,
            "frac_of_floor": round(floor["us_mean"] / head["us_mean"], 4) if floor else None,
            "frac_of_floor_b3": round(floor["us_mean"] / b3["us_mean"], 4) if floor else None,
        },
        "read_floor": floor,
        "cpu_baseline": cpu,
        "gemv_plan_forced": args.gemv_plan,
        "results": results,
        "config3": config3,
        "mlp": mlp,
        "dense_f16": dense,
        "loader": loader,
        "wide": wide,
        "block_vs_sequential": block_seq,
        "kernel_bench": kbench,
        "static_entry": static_entry,
    }
    print(json.dumps(line), flush=True)
    gpu.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Two device handles on one GPU, driven from two host threads at once.

Each handle owns its stream, workspaces, plan caches and slot epochs; what
the handles share (the kernels' dynamic-LDS limits, the occupancy caches of
the planners, the GPU itself) is guarded. Each thread runs its own mix of
launches (row-band GEMV and block with split sums, the split-K kernel forced
to four splits, dense F16 on the matrix cores with split sums, the wide block,
the fused MLP form over several rounds with two-phase staging and with
elected finishers)
several times in its own order, and every output must equal, bit for bit,
the same launch run alone on the session handle: a launch's sums depend only
on its plan. ctypes releases the GIL around each C call, so the two threads'
encodes and launches overlap.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest

import qmr
from test_zz_no_alloc import _case

pytestmark = pytest.mark.gpu

CASES = [
    # form, forced plan, (rows, cols, batch)
    ("plain", (0, 0), (5120, 17408, 1)),
    ("plain", (0, 0), (5120, 17408, 3)),
    ("plain", (-2, 4), (5120, 17408, 3)),
    ("dense", (0, 0), (5120, 17408, 3)),
    ("dense", (-5, 408), (17408, 5120, 2)),
    ("wide", (0, 0), (2048, 5120, 64)),
    ("mlp", (0, 0), (17408, 5120, 3)),   # band MLP form over several rounds, x in two phases
    ("mlp", (0, 0), (17408, 5120, 4)),   # band MLP form, elected finishers
]


def _run(gpu, bufs, name, params, rows, batch, plan):
    _, threads = qmr.dispatch_layout(name, params)
    gpu.set_gemv_plan(*plan)
    try:
        cmd = gpu.begin()
        try:
            cmd.encode(name, bufs, params, threads, 128)
            cmd.finish()
        finally:
            cmd.release()
    finally:
        gpu.set_gemv_plan(0, 0)
    return gpu.read_f32(bufs[-1], batch * rows)


def _upload(gpu, arrays, rows, batch):
    bufs = [gpu.upload_bytes(np.ascontiguousarray(a)) for a in arrays]
    bufs.append(gpu.upload_f32(np.full(batch * rows, np.nan, np.float32)))
    return bufs


def test_two_handles_on_two_threads_match_lone_launches(gpu):
    rng = np.random.default_rng(31)
    cases = []
    for form, plan, (rows, cols, batch) in CASES:
        name, arrays, params, _ = _case(rng, form, rows, cols, batch)
        cases.append((name, arrays, params, rows, batch, plan))
    alone = []
    for name, arrays, params, rows, batch, plan in cases:
        print(f"alone: {name} {rows}x{params[1]} B={batch} plan {plan}", flush=True)
        alone.append(_run(gpu, _upload(gpu, arrays, rows, batch), name, params, rows, batch, plan))

    results: dict[int, list] = {0: [], 1: []}
    errors: list[BaseException] = []
    start = threading.Barrier(2)

    def worker(tid: int) -> None:
        try:
            h = qmr.Gpu("aligned")
            try:
                bufs = [_upload(h, arrays, rows, batch) for name, arrays, params, rows, batch, plan in cases]
                order = list(range(len(cases)))
                if tid == 1:
                    order.reverse()
                start.wait(timeout=60)
                for rep in range(3):
                    for i in order:
                        name, _, params, rows, batch, plan = cases[i]
                        results[tid].append((i, _run(h, bufs[i], name, params, rows, batch, plan)))
            finally:
                h.close()
        except BaseException as e:  # reported in the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(t,)) for t in (0, 1)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    for tid in (0, 1):
        assert len(results[tid]) == 3 * len(cases)
        for i, got in results[tid]:
            name, _, params, rows, batch, plan = cases[i]
            assert np.array_equal(got.view(np.uint32), alone[i].view(np.uint32)), \
                f"thread {tid}: {name} {rows}x{params[1]} B={batch} plan {plan}"

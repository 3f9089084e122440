"""qmr_encode_static, the no-allocation variant of qmr_encode, on the GPU
through the C ABI. Each kernel family whose launches take workspace (the
row-band kernel's split sums, the split-K kernel's partial sums and counters
in the plain, residual and MLP forms, the wide block's activation images,
the dense F16 matrix-core kernel's split sums and counters) is
run twice in a row through qmr_encode_static, the second call on a smaller
input so that it finds the first call's contents in the shared scratch, and
each output is compared with qmr_encode's on the same inputs (same plan, so
bit-identical) and with the FP64 oracle of the reference's product
(tests/quantized.rs:39-51, tests/batch_matrix.rs:35-49) at the BASELINE gate
(rel-L2 <= 1e-5, max-abs <= 1e-4*max|y64|). A launch whose workspace exceeds
the static scratch is rejected before anything is enqueued.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qmr
import qmr.synth as synth
from helpers import assert_gate

pytestmark = pytest.mark.gpu

EPS = float(np.float32(1e-6))
EPS_BITS = int(np.float32(EPS).view(np.uint32))


def _matrix(rng, rows, cols):
    """Q4/g64 codes with BF16 scales and biases."""
    w = rng.integers(0, 2**32, rows * cols // 8, dtype=np.uint64).astype(np.uint32)
    sf = rng.uniform(0.002, 0.02, rows * cols // 64).astype(np.float32)
    bf = (-8 * sf + rng.normal(0, 1e-3, sf.size)).astype(np.float32)
    return w, synth.f32_to_bf16_bits(sf), synth.f32_to_bf16_bits(bf)


def _case(rng, form, rows, cols, batch):
    """Inputs of one launch: (name, host arrays in buffer order, params, FP64 oracle)."""
    if form == "dense":
        w16 = rng.standard_normal(rows * cols).astype(np.float16).view(np.uint16)
        x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
        want = oracle.dense_f16_f64(w16, x, rows, cols, batch)
        if batch == 1:
            return "matvec_f16", [w16, x.ravel()], [rows, cols], want
        return "matmul_f16", [w16, x.ravel()], [rows, cols, batch], want
    m = _matrix(rng, rows, cols)
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    params = [rows, cols, 4, 64, batch]
    if form == "mlp":
        up = _matrix(rng, rows, cols)
        nw = rng.uniform(0.2, 1.8, cols).astype(np.float32)
        want = oracle.mlp_gate_up_f64(m, up, "bf16", x, nw, EPS, rows, cols, 4, 64, batch, 8)
        return "mlp_gate_up_swiglu_bf16", [*m, *up, x.ravel(), nw], params + [EPS_BITS], want
    want = oracle.matmul_f64(*m, "bf16", x, rows, cols, 4, 64, batch, 16)
    if form == "residual":
        r = rng.normal(0, 1, batch * rows).astype(np.float32)
        return "matmul_affine_add_bf16", [*m, x.ravel(), r], params, want + r.astype(np.float64)
    if form == "wide":
        return "matmul_affine_wide_bf16", [*m, x.ravel()], params, want
    if batch == 1:
        return "matvec_affine_bf16", [*m, x.ravel()], params[:4], want
    return "matmul_affine_bf16", [*m, x.ravel()], params, want


def _launch(gpu, name, arrays, params, rows, batch, static, plan):
    """One launch in its own command; returns (y, the HIP kernel that ran)."""
    bufs = [gpu.upload_bytes(np.ascontiguousarray(a)) for a in arrays]
    bufs.append(gpu.upload_f32(np.full(batch * rows, np.nan, np.float32)))
    _, threads = qmr.dispatch_layout(name, params)
    gpu.set_gemv_plan(*plan)
    try:
        cmd = gpu.begin()
        cmd.encode(name, bufs, params, threads, 128, static_scratch=static)
        cmd.finish()
        cmd.release()
        kernel = gpu.last_hip_kernel()
    finally:
        gpu.set_gemv_plan(0, 0)
    return gpu.read_f32(bufs[-1], batch * rows), kernel


# form, forced plan, the first call's shape, the second (smaller) call's
# shape, both (rows, cols, batch), and the kernel the first call must take.
CASES = [
    ("plain", (0, 0), (5120, 17408, 3), (2048, 8192, 2), "affine_band_kernel"),      # split sums
    ("plain", (0, 0), (17408, 5120, 4), (1000, 4096, 1), "affine_band_kernel"),
    ("plain", (-4, 240202), (5120, 17408, 1), (2048, 8192, 4), "affine_band_kernel"),  # 4 splits forced
    ("plain", (-2, 0), (17408, 5120, 2), (4096, 2048, 1), "affine_mfma_kernel"),      # partials + counters
    ("residual", (0, 0), (5120, 17408, 2), (1024, 4096, 1), "affine_band_kernel"),   # y = r + W x
    ("mlp", (0, 0), (4096, 2048, 3), (512, 1024, 1), "affine_band_kernel"),          # gate and up sums
    ("mlp", (-2, 0), (4096, 2048, 3), (512, 1024, 1), "affine_mfma_kernel (MLP)"),
    ("wide", (0, 0), (2048, 5120, 64), (512, 2048, 16), "wide_mfma_kernel"),         # activation images
    ("dense", (0, 0), (5120, 17408, 3), (2048, 8192, 2), "dense_mfma_kernel"),       # dense F16 split sums
    ("dense", (-5, 408), (17408, 5120, 4), (1000, 4096, 2), "dense_mfma_kernel"),
]


@pytest.mark.parametrize("form,plan,first,second,family", CASES)
def test_static_entry_matches_qmr_encode_on_two_calls_in_a_row(gpu, form, plan, first, second, family):
    """The static calls run on a device handle opened here, which has never
    grown a workspace: after them it still holds none, so the calls could
    only have used the static scratch. qmr_encode runs on the session handle."""
    rng = np.random.default_rng([len(form), *first, *second])
    cases = [_case(rng, form, *shape) for shape in (first, second)]
    static = []
    fresh = qmr.Gpu("aligned")
    try:
        assert fresh.workspace_bytes() == 0
        for (rows, _, batch), (name, arrays, params, _) in zip((first, second), cases):
            print(f"qmr_encode_static {name} {rows}x{params[1]} B={batch} plan {plan}", flush=True)
            static.append(_launch(fresh, name, arrays, params, rows, batch, True, plan))
        assert fresh.workspace_bytes() == 0, fresh.workspace_bytes()
    finally:
        fresh.close()
    # The first call takes a kernel with workspace (split sums when banded).
    kernel = static[0][1]
    assert kernel.startswith(family), (kernel, family)
    if form != "mlp":  # the band kernel's MLP form uses its slots at any split count
        assert " ns=1 " not in kernel, kernel
    for (rows, _, batch), (name, arrays, params, want), (got, kernel) in zip((first, second), cases, static):
        ref, ref_kernel = _launch(gpu, name, arrays, params, rows, batch, False, plan)
        label = f"{form} {rows}x{params[1]} B={batch} ({kernel})"
        assert kernel == ref_kernel, (kernel, ref_kernel)
        assert np.isfinite(got).all(), label
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), label
        assert_gate(got, want, label)


def test_static_band_slots_stay_clear_across_a_sequence_of_calls(gpu):
    """GEMVs and blocks on the row-band kernel and every split-K launch clear
    the split-sum slots (and counters) they take, so consecutive static calls
    skip the fill; the row-band MLP form leaves its slots to be cleared
    again, over their whole extent: a GEMV that needs fewer slots than the
    MLP form left behind, followed by a block that needs more, must not find
    the MLP form's sums in the part the GEMV did not clear. Every call of a
    mixed sequence must match qmr_encode bit for bit."""
    rng = np.random.default_rng(23)
    seq = [("plain", (0, 0), (5120, 17408, 1)), ("plain", (0, 0), (5120, 17408, 3)),
           ("residual", (0, 0), (2048, 8192, 2)), ("plain", (-4, 240202), (4096, 8192, 1)),
           ("mlp", (0, 0), (1024, 2048, 2)), ("plain", (0, 0), (5120, 17408, 2)),
           ("plain", (-2, 0), (4096, 2048, 1)), ("plain", (0, 0), (5120, 17408, 1)),
           ("plain", (0, 0), (5120, 17408, 1)),
           # MLP slots (2 splits x 2 matrices x 3 RHS x 4096 rows x 8 bytes)
           # beyond a GEMV's (3 x 5120 x 8) but not a 3-RHS block's.
           ("mlp", (-4, 220202), (4096, 2048, 3)), ("plain", (0, 0), (5120, 17408, 1)),
           ("plain", (0, 0), (5120, 17408, 3)),
           # Split-K's MLP form and a forced four-way split, then the band.
           ("mlp", (-2, 0), (4096, 2048, 3)), ("plain", (-2, 4), (5120, 17408, 3)),
           ("plain", (0, 0), (5120, 17408, 3)),
           # Elected finishers: slots of every split, then the arrival counters.
           ("plain", (-4, 240801), (40960, 2048, 2)), ("plain", (-4, 240801), (40960, 2048, 2)),
           ("plain", (0, 0), (5120, 17408, 1)),
           # Dense F16 split sums after an MLP form left its slots, then the band.
           ("mlp", (-4, 220202), (4096, 2048, 3)), ("dense", (-5, 408), (5120, 17408, 3)),
           ("dense", (0, 0), (17408, 5120, 2)), ("plain", (0, 0), (5120, 17408, 3))]
    fresh = qmr.Gpu("aligned")
    try:
        for form, plan, (rows, cols, batch) in seq:
            name, arrays, params, want = _case(rng, form, rows, cols, batch)
            print(f"sequence: qmr_encode_static {name} {rows}x{cols} B={batch} plan {plan}", flush=True)
            got, kernel = _launch(fresh, name, arrays, params, rows, batch, True, plan)
            ref, ref_kernel = _launch(gpu, name, arrays, params, rows, batch, False, plan)
            label = f"{form} {rows}x{cols} B={batch} ({kernel})"
            assert kernel == ref_kernel, (kernel, ref_kernel)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), label
            assert_gate(got, want, label)
        assert fresh.workspace_bytes() == 0, fresh.workspace_bytes()
    finally:
        fresh.close()


def test_static_entry_rejects_workspace_beyond_the_scratch(gpu):
    """A wide block of 256 RHS over 17408 columns needs 272*8 images of 8448
    bytes (18.4 MB) against the 8 MiB scratch: rejected, nothing enqueued
    (the output keeps its contents), while qmr_encode runs it."""
    rng = np.random.default_rng(9)
    rows, cols, batch = 64, 17408, 256
    name, arrays, params, want = _case(rng, "wide", rows, cols, batch)
    bufs = [gpu.upload_bytes(np.ascontiguousarray(a)) for a in arrays]
    y = gpu.upload_f32(np.full(batch * rows, 7.0, np.float32))
    _, threads = qmr.dispatch_layout(name, params)
    cmd = gpu.begin()
    with pytest.raises(qmr.QmrError) as err:
        cmd.encode(name, bufs + [y], params, threads, 128, static_scratch=True)
    cmd.finish()
    cmd.release()
    assert err.value.code == qmr.QMR_ERR_INVALID
    assert "static scratch" in str(err.value) and str(qmr.STATIC_SCRATCH_BYTES) in str(err.value)
    assert np.all(gpu.read_f32(y, batch * rows) == 7.0)
    gpu.dispatch(name, bufs + [y], params)
    assert_gate(gpu.read_f32(y, batch * rows), want, "qmr_encode wide 256")

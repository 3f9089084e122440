"""A launch whose last K split gives up waiting must fail its command.

The row-band kernel's last split waits (boundedly) for the other splits'
sums; if a band's workgroups were not all resident at once it gives up,
writes NaN for the band and sets the device's status word, and
qmr_command_finish returns QMR_ERR_DEVICE naming the kernel and band, as the
reference fails a frame whose Metal command buffer did not complete
(src/gpu.rs:861-865). The split-K kernel's last arriver waits the same way
for each partial's epoch tag and reports the same way, and so does the dense
F16 matrix-core kernel's.

The give-up is forced from the host (qmr_set_band_wait_fault: the last
arrivers wait for a tag that no split of the launch publishes, with a short
bound), so every workgroup still exits normally. After the failed command the
same device runs the next command correctly, through qmr_encode and through
qmr_encode_static, whose scratch the failure leaves to be cleared again.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qmr
from helpers import assert_gate
from test_zz_no_alloc import EPS, EPS_BITS, _matrix

pytestmark = pytest.mark.gpu


def _inputs(rng, rows, cols, batch, form):
    if form == "dense":
        w16 = rng.standard_normal(rows * cols).astype(np.float16).view(np.uint16)
        x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
        want = oracle.dense_f16_f64(w16, x, rows, cols, batch)
        return "matmul_f16", [w16, x.ravel()], [rows, cols, batch], want
    m = _matrix(rng, rows, cols)
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    if form == "mlp":
        up = _matrix(rng, rows, cols)
        nw = rng.uniform(0.2, 1.8, cols).astype(np.float32)
        want = oracle.mlp_gate_up_f64(m, up, "bf16", x, nw, EPS, rows, cols, 4, 64, batch, 8)
        return ("mlp_gate_up_swiglu_bf16", [*m, *up, x.ravel(), nw], [rows, cols, 4, 64, batch, EPS_BITS], want)
    want = oracle.matmul_f64(*m, "bf16", x, rows, cols, 4, 64, batch, 16)
    if batch == 1:
        return "matvec_affine_bf16", [*m, x.ravel()], [rows, cols, 4, 64], want
    return "matmul_affine_bf16", [*m, x.ravel()], [rows, cols, 4, 64, batch], want


def _command(gpu, name, bufs, params, static):
    _, threads = qmr.dispatch_layout(name, params)
    cmd = gpu.begin()
    try:
        cmd.encode(name, bufs, params, threads, 128, static_scratch=static)
        cmd.finish()
    finally:
        cmd.release()


@pytest.mark.parametrize("static", [False, True])
@pytest.mark.parametrize("rows,cols,batch,form,plan,kernel", [
    (5120, 17408, 1, "plain", (0, 0), "affine_band_kernel"),      # the metric shape's default plan: three K splits
    (5120, 17408, 3, "plain", (0, 0), "affine_band_kernel"),
    (4096, 2048, 3, "mlp", (-4, 220202), "affine_band_kernel"),   # the MLP form with two K splits
    (5120, 17408, 3, "plain", (-2, 4), "affine_mfma_kernel"),     # split-K, four K splits
    (4096, 2048, 3, "mlp", (-2, 0), "affine_mfma_kernel"),        # split-K's MLP form
    (40960, 2048, 2, "plain", (-4, 240801), "affine_band_kernel"),  # elected finishers, several rounds
    (5120, 17408, 3, "dense", (-5, 408), "dense_mfma_kernel"),    # dense F16, eight K splits
])
def test_give_up_fails_the_command_and_the_next_one_succeeds(gpu, static, rows, cols, batch, form, plan, kernel):
    rng = np.random.default_rng([rows, cols, batch, int(static)])
    name, arrays, params, want = _inputs(rng, rows, cols, batch, form)
    bufs = [gpu.upload_bytes(np.ascontiguousarray(a)) for a in arrays]
    y = gpu.upload_f32(np.zeros(batch * rows, np.float32))
    print(f"wait fault {name} {rows}x{cols} B={batch} static={static}", flush=True)
    gpu.set_gemv_plan(*plan)
    try:
        gpu.set_band_wait_fault(True)
        try:
            with pytest.raises(qmr.QmrError) as err:
                _command(gpu, name, bufs + [y], params, static)
        finally:
            gpu.set_band_wait_fault(False)
        assert err.value.code == qmr.QMR_ERR_DEVICE, err.value
        assert f"{kernel} band" in str(err.value), str(err.value)
        assert gpu.last_hip_kernel().startswith(kernel), gpu.last_hip_kernel()
        assert " ns=1 " not in gpu.last_hip_kernel(), gpu.last_hip_kernel()
        assert np.isnan(gpu.read_f32(y, batch * rows)).any()
        # The next command on the same device: correct, and its finish succeeds.
        _command(gpu, name, bufs + [y], params, static)
    finally:
        gpu.set_gemv_plan(0, 0)
    assert_gate(gpu.read_f32(y, batch * rows), want, f"after the failed command ({name}, static={static})")
    # A command with no band launch after it also finishes cleanly.
    gpu.dispatch("copy_f32", [y, gpu.alloc_f32(batch * rows)], [batch * rows])

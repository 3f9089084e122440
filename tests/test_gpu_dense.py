"""Dense F16 products (matvec_f16 / matmul_f16, kernels/qwen.metal:48-57,
kernels/matmul_block.metal:213-248) on the matrix-core kernel against the
FP64 oracle, at the BASELINE gate (rel-L2 <= 1e-5, max-abs <= 1e-4*max|y64|):
the planner's plans at the decoder's dense shapes, every workgroup shape and
a range of K split counts forced on one small matrix with row and column
tails, outputs at an offset between guard values, x over a wide dynamic range
against a per-row error bound, the static-scratch entry point (bit-identical
to qmr_encode, twice in a row), and the routing rules (unaligned weights,
cols % 32 != 0, one RHS by default, products whose plan the planner
estimates slower than the vector-ALU kernel, and the rr = -1 hook take the
vector-ALU kernels)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qmr
from helpers import assert_gate

pytestmark = pytest.mark.gpu

MAX_SPLITS = 32


def _dense(rng, rows, cols, batch):
    w16 = rng.standard_normal(rows * cols).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    return w16, x


def _name(batch):
    return "matvec_f16" if batch == 1 else "matmul_f16"


def _params(rows, cols, batch):
    return [rows, cols] + ([batch] if batch > 1 else [])


def _label(ks):
    """The HIP kernel label of a dense plan code (ring*10000 + kw*1000 +
    rt*100 + ns)."""
    return f"dense_mfma_kernel ring={ks // 10000} kw={ks // 1000 % 10} rt={ks // 100 % 10} ns={ks % 100}"


def _run(gpu, w16, x, rows, cols, batch, static=False, w_offset=0):
    """One dense product in its own command (weights at `w_offset` bytes, y
    between guards); returns (y, the HIP kernel that ran)."""
    wb = gpu.upload_bytes(np.concatenate([np.zeros(w_offset // 2, np.uint16), w16]))
    xb = gpu.upload_f32(np.concatenate([[99.0], x.ravel()]).astype(np.float32))
    yb = gpu.upload_f32(np.full(batch * rows + 2, 12345.0, np.float32))
    params = _params(rows, cols, batch)
    _, threads = qmr.dispatch_layout(_name(batch), params)
    cmd = gpu.begin()
    try:
        cmd.encode(_name(batch), [wb, xb, yb], params, threads, 128, [w_offset, 4, 4], static_scratch=static)
        cmd.finish()
    finally:
        cmd.release()
    got = gpu.read_f32(yb, batch * rows + 2)
    assert got[0] == 12345.0 and got[-1] == 12345.0, "wrote outside y"
    return got[1:-1], gpu.last_hip_kernel()


@pytest.mark.parametrize("rows,cols", [(5120, 17408), (17408, 5120), (5120, 5120), (1024, 1024), (4096, 2048)])
@pytest.mark.parametrize("batch", [1, 2, 3, 4])
@pytest.mark.parametrize("forced", [False, True])
def test_planner_plans_on_decoder_shapes(gpu, rows, cols, batch, forced):
    """The default choice (the matrix-core kernel for two or more RHS where
    its planner's estimate beats the vector-ALU kernel's; the vector-ALU
    kernels for one RHS) and, with rr = -5, the matrix-core planner's own
    plan, as qmr_gemv_plan reports them."""
    rng = np.random.default_rng([rows, cols, batch])
    w16, x = _dense(rng, rows, cols, batch)
    print(f"dense {rows}x{cols} B={batch} forced={forced}", flush=True)
    gpu.set_gemv_plan(-5 if forced else 0, 0)
    try:
        got, kernel = _run(gpu, w16, x, rows, cols, batch)
        rr, ks = gpu.gemv_plan(rows, cols, 16, batch)
    finally:
        gpu.set_gemv_plan(0, 0)
    if forced or rr == -5:
        assert rr == -5 and kernel == _label(ks), (rr, ks, kernel)
    else:
        assert rr == -1 and kernel == "dense_f16_kernel", (rr, ks, kernel)
    if not forced and batch == 1:
        assert rr == -1
    if not forced and (rows, cols) in ((5120, 17408), (17408, 5120)) and batch > 1:
        assert rr == -5, "the matrix-core kernel is the faster one here at 2-4 RHS"
    assert_gate(got, oracle.dense_f16_f64(w16, x, rows, cols, batch), f"dense {rows}x{cols} B{batch} {kernel}")


def _feasible(rows, cols, batch, ring, kw, rt, ns, max_lds):
    tiles = -(-cols // 128)
    if ns > tiles or ns > MAX_SPLITS or (rt > -(-rows // 16) and rt > 1) or rt * kw > 8:
        return False
    tps = -(-tiles // ns)
    if -(-tiles // tps) != ns or kw > tps:
        return False
    threads = rt * kw * 64
    xi = -(-(tps * batch * 16) // threads)
    lds = tps * (512 * batch + 64) + threads * 8 + 16
    return xi <= 8 and lds <= max_lds


@pytest.mark.parametrize("batch", [1, 2, 3, 4])
def test_forced_shapes_and_split_counts(gpu, batch):
    """300 rows (18 full 16-row tiles and a 12-row tail) x 4192 columns (32
    full 128-column tiles and a 96-column tail): both ring depths, workgroups
    of one to eight row tiles and one to eight K runs per tile, and one to
    seventeen K splits, each against the oracle; shapes the kernel cannot
    hold fall back to its planner's plan."""
    rows, cols = 300, 4192
    rng = np.random.default_rng([rows, cols, batch, 7])
    w16, x = _dense(rng, rows, cols, batch)
    want = oracle.dense_f16_f64(w16, x, rows, cols, batch)
    gpu.set_gemv_plan(-5, 0)
    default = gpu.gemv_plan(rows, cols, 16, batch)
    ran = set()
    try:
        for ring in (4, 8):
            for kw, rt in ((1, 1), (2, 1), (8, 1), (1, 2), (4, 2), (2, 4), (1, 8)):
                for ns in (1, 2, 3, 5, 11, 17):
                    code = ring * 10000 + kw * 1000 + rt * 100 + ns
                    gpu.set_gemv_plan(-5, code)
                    plan = gpu.gemv_plan(rows, cols, 16, batch)
                    if _feasible(rows, cols, batch, ring, kw, rt, ns, gpu.max_lds()):
                        assert plan == (-5, code), (code, plan)
                    else:
                        assert plan == default, (code, plan, default)
                    print(f"dense forced {code} B={batch}", flush=True)
                    got, kernel = _run(gpu, w16, x, rows, cols, batch)
                    assert kernel == _label(plan[1]), (kernel, plan)
                    assert_gate(got, want, f"dense forced {kernel} B{batch}")
                    ran.add(plan[1])
    finally:
        gpu.set_gemv_plan(0, 0)
    assert len(ran) >= 40, sorted(ran)


@pytest.mark.parametrize("rows", [1, 15, 17, 77])
@pytest.mark.parametrize("cols", [32, 96, 160, 1056])
def test_row_and_column_tails_keep_guards(gpu, rows, cols):
    rng = np.random.default_rng([rows, cols])
    for batch in (1, 2, 3, 4):
        w16, x = _dense(rng, rows, cols, batch)
        want = oracle.dense_f16_f64(w16, x, rows, cols, batch)
        for w_offset in (0, 16):
            gpu.set_gemv_plan(-5, 0)
            try:
                got, kernel = _run(gpu, w16, x, rows, cols, batch, w_offset=w_offset)
            finally:
                gpu.set_gemv_plan(0, 0)
            assert kernel.startswith("dense_mfma_kernel"), kernel
            assert_gate(got, want, f"dense tail {rows}x{cols} B{batch} w+{w_offset}")


def test_routing_to_the_vector_alu_kernels(gpu):
    """Weights off a 16-byte boundary, rows with cols % 32 != 0 and the
    rr = -1 hook use the vector-ALU kernels; results still meet the gate."""
    rng = np.random.default_rng(5)
    for rows, cols, batch, w_offset, plan in [(64, 1024, 2, 4, (0, 0)), (64, 1000, 3, 0, (0, 0)),
                                              (64, 1024, 4, 0, (-1, 0)), (640, 5120, 1, 8, (0, 0))]:
        w16, x = _dense(rng, rows, cols, batch)
        gpu.set_gemv_plan(*plan)
        try:
            got, kernel = _run(gpu, w16, x, rows, cols, batch, w_offset=w_offset)
        finally:
            gpu.set_gemv_plan(0, 0)
        assert kernel == "dense_f16_kernel", (rows, cols, w_offset, plan, kernel)
        assert_gate(got, oracle.dense_f16_f64(w16, x, rows, cols, batch), f"dense VALU {rows}x{cols}")
    gpu.set_gemv_plan(-5, 0)
    try:
        assert gpu.gemv_plan(64, 1024, 16, 1)[0] == -5
    finally:
        gpu.set_gemv_plan(0, 0)
    gpu.set_gemv_plan(-1, 0)
    try:
        assert gpu.gemv_plan(64, 1024, 16, 1) == (-1, 0)
    finally:
        gpu.set_gemv_plan(0, 0)


@pytest.mark.parametrize("plan", [(-5, 0), (-5, 405)])
def test_wide_dynamic_range_meets_a_per_row_bound(gpu, plan):
    """x spans 2^-24 .. 2^24 inside every 128-column tile and the weights
    include F16 subnormals and +-65504. Each x element reaches the matrix
    core as hi + lo f16 parts scaled by a power of two per (tile, RHS), which
    carries x to within 2^-22 of the tile's max |x| (the scaled max sits in
    [2^14, 2^15), where hi's rounding error is at most 8 and lo's relative
    error 2^-11); the products are exact, and FP32 accumulation rounds at
    most 24 times inside a tile's four MFMAs (a five-level adder tree and the
    accumulator, each) and once per tile, split and final add outside. So per
    row and RHS
        |y - y64| <= (2^-21 + (tiles + 32) 2^-24) * sum_c |w_c| M(c)
    with M(c) the max |x| of c's tile. A misplaced column or a wrong scale
    exceeds it."""
    rows, cols, batch = 333, 5120, 4
    rng = np.random.default_rng(11)
    mag = np.exp2(rng.integers(-24, 25, (batch, cols))).astype(np.float32)
    x = (mag * rng.choice([-1.0, 1.0], (batch, cols)) * rng.uniform(1, 2, (batch, cols))).astype(np.float32)
    w = rng.standard_normal(rows * cols).astype(np.float16)
    special = rng.random(rows * cols)
    w[special < 0.01] = np.float16(65504.0)
    w[(special >= 0.01) & (special < 0.02)] = np.float16(-65504.0)
    w[(special >= 0.02) & (special < 0.05)] = (rng.integers(1, 1024, int(((special >= 0.02) & (special < 0.05)).sum()))
                                               .astype(np.uint16).view(np.float16))
    w16 = w.view(np.uint16)
    gpu.set_gemv_plan(*plan)
    try:
        got, kernel = _run(gpu, w16, x, rows, cols, batch)
    finally:
        gpu.set_gemv_plan(0, 0)
    assert kernel.startswith("dense_mfma_kernel"), kernel
    want = oracle.dense_f16_f64(w16, x, rows, cols, batch).reshape(batch, rows)
    tiles = -(-cols // 128)
    tile_max = np.repeat(np.abs(x.astype(np.float64)).reshape(batch, tiles, 128).max(axis=2), 128, axis=1)
    wabs = np.abs(w.astype(np.float64)).reshape(rows, cols)
    bound = (2.0**-21 + (tiles + 32) * 2.0**-24) * (tile_max @ wabs.T)
    err = np.abs(got.reshape(batch, rows).astype(np.float64) - want)
    worst = float(np.max(err / bound))
    assert worst <= 1.0, f"{kernel}: error reaches {worst:.3f} of the per-row bound"


def test_static_scratch_is_bit_identical_twice_in_a_row(gpu):
    """qmr_encode_static runs the same plan as qmr_encode with its split sums
    and counters in the GPU's static scratch; two calls in a row (the second
    smaller, finding the first's region) each give qmr_encode's bits."""
    rng = np.random.default_rng(3)
    for rows, cols, batch, plan in [(5120, 17408, 3, (-5, 408)), (1000, 4096, 2, (-5, 206)),
                                    (5120, 17408, 2, (0, 0))]:
        w16, x = _dense(rng, rows, cols, batch)
        gpu.set_gemv_plan(*plan)
        try:
            ref, k1 = _run(gpu, w16, x, rows, cols, batch)
            got, k2 = _run(gpu, w16, x, rows, cols, batch, static=True)
        finally:
            gpu.set_gemv_plan(0, 0)
        assert k1 == k2 and k1.startswith("dense_mfma_kernel"), (k1, k2)
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), f"static {rows}x{cols} {k1}"
        assert_gate(got, oracle.dense_f16_f64(w16, x, rows, cols, batch), f"static {k1}")


def test_static_scratch_too_small_for_the_split_sums_takes_the_vector_alu_kernel(gpu):
    """A plan whose split sums exceed the static scratch (here eight splits
    of 4 x 65536 outputs: 16.8 MB against 8 MiB) runs, under
    qmr_encode_static, on the vector-ALU kernel, which needs no workspace;
    qmr_encode keeps the matrix-core plan. Both meet the gate."""
    rows, cols, batch = 65536, 2048, 4
    rng = np.random.default_rng(21)
    w16, x = _dense(rng, rows, cols, batch)
    want = oracle.dense_f16_f64(w16, x, rows, cols, batch)
    gpu.set_gemv_plan(-5, 408)
    try:
        got, kernel = _run(gpu, w16, x, rows, cols, batch)
        assert kernel.startswith("dense_mfma_kernel") and kernel.endswith(" rt=4 ns=8"), kernel
        assert_gate(got, want, "dense 8 splits, qmr_encode")
        got, kernel = _run(gpu, w16, x, rows, cols, batch, static=True)
        assert kernel == "dense_f16_kernel", kernel
        assert_gate(got, want, "dense, qmr_encode_static fallback")
    finally:
        gpu.set_gemv_plan(0, 0)


def test_repeated_launches_reuse_slots(gpu):
    """Split plans tag their sums with a new epoch per launch over the same
    slot workspace: repeated launches with different inputs each give their
    own product."""
    rows, cols, batch = 2048, 8192, 2
    rng = np.random.default_rng(9)
    gpu.set_gemv_plan(-5, 416)
    try:
        for i in range(4):
            w16, x = _dense(rng, rows, cols, batch)
            got, kernel = _run(gpu, w16, x, rows, cols, batch)
            assert kernel.startswith("dense_mfma_kernel") and kernel.endswith(" rt=4 ns=16"), kernel
            assert_gate(got, oracle.dense_f16_f64(w16, x, rows, cols, batch), f"launch {i}")
    finally:
        gpu.set_gemv_plan(0, 0)

"""The row-band matrix-core kernel (affine_tile.hip) on the GPU through the C
ABI, against the FP64 oracle of the reference's per-weight product
(tests/quantized.rs:39-51, tests/batch_matrix.rs:35-49) with the BASELINE
gate (rel-L2 <= 1e-5, max-abs <= 1e-4*max|y64|).

Every shape is run under plans forced through the tuning hook (rr = -4,
ks = phases*1000000 + ring*100000 + ns*10000 + tr*100 + kw, phases 0 for the
planner's choice) so that each code path is taken:
one to eight K splits (the last split adds the others' epoch-tagged sums),
one to eight row tiles per band, one to eight waves per tile, two- and
three-entry rings, x staged in one or two phases; row tails, K tails that end inside a tile or inside a
128-byte entry, Q8, groups 32/64/128, F32/BF16/F16 metadata, and metadata
runs that are not 16-byte multiples (per-value staging path).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import qmr
import qmr.synth as synth
from helpers import assert_gate

pytestmark = pytest.mark.gpu

SUFFIX = {"bf16": "_bf16", "f16": "_f16meta", "f32": ""}


def _matrix(rng, rows, cols, bits, group, kind):
    pack = 32 // bits
    w = rng.integers(0, 2**32, rows * cols // pack, dtype=np.uint64).astype(np.uint32)
    levels = (1 << bits) - 1
    sf = rng.uniform(0.002, 0.02, rows * cols // group).astype(np.float32)
    bf = (-(levels + 1) / 2 * sf + rng.normal(0, 1e-3, sf.size)).astype(np.float32)
    if kind == "bf16":
        return w, synth.f32_to_bf16_bits(sf), synth.f32_to_bf16_bits(bf)
    if kind == "f16":
        return w, sf.astype(np.float16).view(np.uint16), bf.astype(np.float16).view(np.uint16)
    return w, sf, bf


def _ks(ring, ns, tr, kw):
    return ring * 100000 + ns * 10000 + tr * 100 + kw


def _run(gpu, m, x, rows, cols, bits, group, batch, kind, plan):
    name = ("matvec_affine" if batch == 1 else "matmul_affine") + SUFFIX[kind]
    bufs = [gpu.upload_bytes(np.ascontiguousarray(a)) for a in m]
    xb = gpu.upload_f32(np.ascontiguousarray(x, np.float32).ravel())
    yb = gpu.upload_f32(np.full(batch * rows, np.nan, np.float32))
    params = [rows, cols, bits, group] + ([batch] if batch > 1 else [])
    gpu.set_gemv_plan(*plan)
    try:
        gpu.dispatch(name, [*bufs, xb, yb], params)
        kernel = gpu.last_hip_kernel()
    finally:
        gpu.set_gemv_plan(0, 0)
    return gpu.read_f32(yb, batch * rows), kernel


CASES = [
    # rows, cols, bits, group, batch, kind
    (5120, 17408, 4, 64, 1, "bf16"),   # the metric shape
    (5120, 17408, 4, 64, 3, "bf16"),   # the metric block
    (17408, 5120, 4, 64, 2, "bf16"),   # gate/up, two RHS
    (300, 4160, 4, 64, 2, "f32"),      # row tail; K ends inside a tile and an entry
    (1000, 5120, 8, 64, 1, "f16"),     # Q8, F16 metadata
    (72, 2048, 4, 128, 4, "bf16"),     # group 128, four RHS, 4.5 row tiles
    (24, 4096, 8, 32, 2, "bf16"),      # group 32, fewer rows than two tiles
    (260, 576, 4, 64, 1, "bf16"),      # 9 groups per row: per-value metadata staging
    (129, 1152, 8, 128, 3, "f32"),     # Q8/g128 FP32 metadata, one row past a tile
    (96, 5120, 8, 128, 2, "bf16"),     # Q8/g128: three splits start at entries 13 and 26, so the
                                       # 16-bit metadata runs start 5 and 2 groups past a 16-byte unit
]
PLANS = [(2, 1, 1, 1), (3, 1, 2, 2), (2, 2, 4, 2), (3, 3, 4, 2), (3, 4, 2, 4), (2, 3, 8, 1), (2, 2, 1, 8)]


@pytest.mark.parametrize("rows,cols,bits,group,batch,kind", CASES)
def test_band_plans_match_fp64_oracle(gpu, rows, cols, bits, group, batch, kind):
    rng = np.random.default_rng([rows, cols, bits, group, batch])
    m = _matrix(rng, rows, cols, bits, group, kind)
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    want = oracle.matmul_f64(*m, kind, x, rows, cols, bits, group, batch, 16)
    band = set()
    for ring, ns, tr, kw in [(0, 0, 0, 0)] + PLANS:
        plan = (-4, _ks(ring, ns, tr, kw)) if ring else (0, 0)
        got, kernel = _run(gpu, m, x, rows, cols, bits, group, batch, kind, plan)
        assert np.isfinite(got).all(), f"plan {plan} ({kernel}): non-finite output"
        assert_gate(got, want, f"{rows}x{cols} Q{bits}/g{group} {kind} B={batch} plan {plan} ({kernel})")
        if kernel.startswith("affine_band_kernel"):
            band.add(kernel)
    # Infeasible forced shapes fall back to other kernels; enough distinct
    # band-kernel plans must have run for the case to test the band kernel.
    assert len(band) >= 3, band
    assert any(" ns=1 " not in k for k in band) or rows * cols < 2**20, band


def test_forced_band_plans_are_taken(gpu):
    """The tuning hook reports the band kernel with the forced shape for the
    metric matrix (the report covers group 64 with BF16 metadata)."""
    for ring, ns, tr, kw in [(3, 3, 4, 2), (2, 3, 4, 2), (3, 3, 2, 2), (2, 4, 2, 2)]:
        gpu.set_gemv_plan(-4, _ks(ring, ns, tr, kw))
        try:
            rr, ks = gpu.gemv_plan(5120, 17408, 4, 1)
        finally:
            gpu.set_gemv_plan(0, 0)
        assert (rr, ks) == (-4, _ks(ring, ns, tr, kw)), (ring, ns, tr, kw, rr, ks)


@pytest.mark.parametrize("rows,cols", [(5120, 17408), (17408, 5120)])
@pytest.mark.parametrize("batch", [1, 2, 3, 4])
def test_default_plan_is_the_band_kernel_at_the_mlp_shapes(gpu, rows, cols, batch):
    rr, ks = gpu.gemv_plan(rows, cols, 4, batch)
    assert rr == -4, (rows, cols, batch, rr, ks)


def test_split_sums_stay_correct_across_back_to_back_launches_of_different_shapes(gpu):
    """Launches of different shapes and split counts share the slot
    workspace; each launch's last split must take only its own launch's sums
    (the epoch tag). Results are bit-identical to isolated launches."""
    rng = np.random.default_rng(7)
    shapes = [(5120, 17408, 3, (3, 3, 4, 2)), (2048, 8192, 1, (2, 4, 2, 2)), (5120, 17408, 3, (3, 2, 4, 2)),
              (777, 4096, 2, (2, 3, 1, 4))]
    mats, xs, isolated = [], [], []
    for rows, cols, batch, (ring, ns, tr, kw) in shapes:
        m = _matrix(rng, rows, cols, 4, 64, "bf16")
        x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
        mats.append(m)
        xs.append(x)
        got, kernel = _run(gpu, m, x, rows, cols, 4, 64, batch, "bf16", (-4, _ks(ring, ns, tr, kw)))
        assert kernel == f"affine_band_kernel ring={ring} ns={ns} tr={tr} kw={kw}", kernel
        isolated.append(got)
    # The same launches back to back in one command, twice over.
    bufs = []
    for (rows, cols, batch, _), m, x in zip(shapes, mats, xs):
        bufs.append([gpu.upload_bytes(np.ascontiguousarray(a)) for a in m] +
                    [gpu.upload_f32(x.ravel()), gpu.alloc_f32(batch * rows)])
    cmd = gpu.begin()
    for _ in range(2):
        for (rows, cols, batch, (ring, ns, tr, kw)), b in zip(shapes, bufs):
            gpu.set_gemv_plan(-4, _ks(ring, ns, tr, kw))
            name = "matvec_affine_bf16" if batch == 1 else "matmul_affine_bf16"
            params = [rows, cols, 4, 64] + ([batch] if batch > 1 else [])
            cmd.encode(name, b, params, rows * 32, 128)
    gpu.set_gemv_plan(0, 0)
    cmd.finish()
    cmd.release()
    for (rows, cols, batch, plan), b, want_bits, m, x in zip(shapes, bufs, isolated, mats, xs):
        got = gpu.read_f32(b[-1], batch * rows)
        assert np.array_equal(got.view(np.uint32), want_bits.view(np.uint32)), (rows, cols, plan)
        assert_gate(got, oracle.matmul_f64(*m, "bf16", x, rows, cols, 4, 64, batch, 16), f"{rows}x{cols}")


def test_band_kernel_is_deterministic_across_launches(gpu):
    rng = np.random.default_rng(11)
    rows, cols, batch = 5120, 17408, 3
    m = _matrix(rng, rows, cols, 4, 64, "bf16")
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    outs = [_run(gpu, m, x, rows, cols, 4, 64, batch, "bf16", (0, 0))[0] for _ in range(3)]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


@pytest.mark.parametrize("in_place", [False, True])
@pytest.mark.parametrize("ring,ns,tr,kw", [(3, 3, 4, 2), (2, 2, 4, 2)])
def test_band_residual_form(gpu, in_place, ring, ns, tr, kw):
    """matmul_affine_add on the band kernel: y = r + W x, with y == r in place."""
    rng = np.random.default_rng([ring, ns, tr, kw, int(in_place)])
    rows, cols, batch = 5120, 17408, 2
    m = _matrix(rng, rows, cols, 4, 64, "bf16")
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    r = rng.normal(0, 1, batch * rows).astype(np.float32)
    bufs = [gpu.upload_bytes(np.ascontiguousarray(a)) for a in m] + [gpu.upload_f32(x.ravel())]
    rb = gpu.upload_f32(r)
    yb = rb if in_place else gpu.alloc_f32(batch * rows)
    gpu.set_gemv_plan(-4, _ks(ring, ns, tr, kw))
    try:
        gpu.dispatch("matmul_affine_add_bf16", bufs + [rb, yb], [rows, cols, 4, 64, batch])
        kernel = gpu.last_hip_kernel()
    finally:
        gpu.set_gemv_plan(0, 0)
    assert kernel == f"affine_band_kernel ring={ring} ns={ns} tr={tr} kw={kw}", kernel
    got = gpu.read_f32(yb, batch * rows)
    want = oracle.matmul_f64(*m, "bf16", x, rows, cols, 4, 64, batch, 16) + r.astype(np.float64)
    assert_gate(got, want, f"residual in_place={in_place}")


@pytest.mark.parametrize("rows,cols,batch,bits,kind,plan", [
    (40960, 2048, 2, 4, "bf16", (2, 4, 8, 1)),   # 1280 workgroups of 8 waves: several rounds
    (70000, 1152, 3, 8, "f32", (3, 2, 8, 1)),    # Q8 FP32, a row tail
    (24576, 4096, 1, 4, "f16", (2, 3, 4, 2)),
])
def test_elected_finishers_over_several_rounds(gpu, rows, cols, batch, bits, kind, plan):
    """Forced split plans whose workgroups do not fit one round (more than
    four 8-wave workgroups per CU) run with elected finishers: every split
    publishes its sums and the band's last workgroup to arrive (an arrival
    counter) adds them in split order, so no workgroup waits for one that is
    not resident. Against the FP64 oracle, and deterministic."""
    rng = np.random.default_rng([rows, cols, batch])
    m = _matrix(rng, rows, cols, bits, 64, kind)
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    want = oracle.matmul_f64(*m, kind, x, rows, cols, bits, 64, batch, 16)
    print(f"elected finishers {rows}x{cols} Q{bits} {kind} B={batch} plan {plan}", flush=True)
    got, kernel = _run(gpu, m, x, rows, cols, bits, 64, batch, kind, (-4, _ks(*plan)))
    ring, ns, tr, kw = plan
    assert kernel == f"affine_band_kernel ring={ring} ns={ns} tr={tr} kw={kw} elect", kernel
    assert_gate(got, want, f"elected {rows}x{cols} plan {plan}")
    again, _ = _run(gpu, m, x, rows, cols, bits, 64, batch, kind, (-4, _ks(*plan)))
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "launches differ"


def test_elected_finishers_residual_form_in_place(gpu):
    rng = np.random.default_rng(41)
    rows, cols, batch, plan = 40960, 2048, 3, (3, 4, 8, 1)
    m = _matrix(rng, rows, cols, 4, 64, "bf16")
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    r = rng.normal(0, 1, batch * rows).astype(np.float32)
    bufs = [gpu.upload_bytes(np.ascontiguousarray(a)) for a in m] + [gpu.upload_f32(x.ravel())]
    rb = gpu.upload_f32(r)
    gpu.set_gemv_plan(-4, _ks(*plan))
    try:
        gpu.dispatch("matmul_affine_add_bf16", bufs + [rb, rb], [rows, cols, 4, 64, batch])
        kernel = gpu.last_hip_kernel()
    finally:
        gpu.set_gemv_plan(0, 0)
    assert kernel.endswith(" elect"), kernel
    want = oracle.matmul_f64(*m, "bf16", x, rows, cols, 4, 64, batch, 16) + r.astype(np.float64)
    assert_gate(gpu.read_f32(rb, batch * rows), want, "elected residual in place")


PHASED_CASES = [
    # rows, cols, bits, group, batch, kind, ring, tr
    (40960, 2048, 4, 64, 2, "bf16", 2, 8),    # 8 entries: the second half starts at entry 4
    (70000, 1152, 8, 64, 3, "f32", 3, 8),     # Q8 (one tile per entry), a row tail
    (300, 4160, 4, 64, 2, "f32", 3, 4),       # 17 entries, K ends inside a tile and an entry
    (1000, 5120, 8, 64, 1, "f16", 2, 2),      # Q8, F16 metadata, 40 entries
    (72, 2048, 4, 128, 4, "bf16", 3, 2),      # group 128, four RHS, 4.5 row tiles
    (260, 576, 4, 64, 1, "bf16", 2, 8),       # 3 entries: too short for two phases, one phase runs
    (24, 4096, 8, 32, 2, "bf16", 2, 2),       # group 32, fewer rows than two tiles
]


@pytest.mark.parametrize("rows,cols,bits,group,batch,kind,ring,tr", PHASED_CASES)
def test_two_phase_x_staging(gpu, rows, cols, bits, group, batch, kind, ring, tr):
    """Single-split plans of one wave per tile forced to stage x in two
    phases (ks + 2000000): the K tiles of the first half of the entries are
    staged, streamed, then replaced by those of the second half in the same
    LDS. Against the FP64 oracle, and bit-identical to the same plan with
    one phase (ks + 1000000): each tile's product and the order of the sums
    are the same."""
    rng = np.random.default_rng([rows, cols, bits, group, batch, 77])
    m = _matrix(rng, rows, cols, bits, group, kind)
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    want = oracle.matmul_f64(*m, kind, x, rows, cols, bits, group, batch, 16)
    ks = _ks(ring, 1, tr, 1)
    print(f"two-phase {rows}x{cols} Q{bits}/g{group} {kind} B={batch} ring {ring} tr {tr}", flush=True)
    got, kernel = _run(gpu, m, x, rows, cols, bits, group, batch, kind, (-4, 2000000 + ks))
    label = f"affine_band_kernel ring={ring} ns=1 tr={tr} kw=1"
    entries = -(-cols * bits // 8 // 128)
    assert kernel == (label + " phased" if entries >= 4 else label), kernel
    assert_gate(got, want, f"two-phase {rows}x{cols} ({kernel})")
    one, kernel1 = _run(gpu, m, x, rows, cols, bits, group, batch, kind, (-4, 1000000 + ks))
    assert kernel1 == label, kernel1
    assert np.array_equal(got.view(np.uint32), one.view(np.uint32)), "two phases differ from one"


@pytest.mark.parametrize("in_place", [False, True])
def test_two_phase_x_staging_residual_form(gpu, in_place):
    rng = np.random.default_rng([43, int(in_place)])
    rows, cols, batch = 17408, 5120, 3
    m = _matrix(rng, rows, cols, 4, 64, "bf16")
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    r = rng.normal(0, 1, batch * rows).astype(np.float32)
    bufs = [gpu.upload_bytes(np.ascontiguousarray(a)) for a in m] + [gpu.upload_f32(x.ravel())]
    rb = gpu.upload_f32(r)
    yb = rb if in_place else gpu.alloc_f32(batch * rows)
    gpu.set_gemv_plan(-4, 2000000 + _ks(3, 1, 8, 1))
    try:
        gpu.dispatch("matmul_affine_add_bf16", bufs + [rb, yb], [rows, cols, 4, 64, batch])
        kernel = gpu.last_hip_kernel()
    finally:
        gpu.set_gemv_plan(0, 0)
    assert kernel == "affine_band_kernel ring=3 ns=1 tr=8 kw=1 phased", kernel
    want = oracle.matmul_f64(*m, "bf16", x, rows, cols, 4, 64, batch, 16) + r.astype(np.float64)
    assert_gate(gpu.read_f32(yb, batch * rows), want, f"two-phase residual in_place={in_place}")


@pytest.mark.parametrize("rows,cols,batch,kind,plan", [
    (5120, 17408, 3, "bf16", (3, 6, 8, 1)),   # six splits, one round
    (5120, 17408, 1, "bf16", (2, 8, 4, 1)),   # eight splits (two chunks of slot reads)
    (300, 4160, 2, "f32", (3, 5, 2, 2)),      # 17 entries in five splits, row and K tails
    (17408, 5120, 3, "bf16", (2, 7, 8, 1)),   # seven splits over several rounds: elected finishers
])
def test_forced_plans_with_more_than_four_splits(gpu, rows, cols, batch, kind, plan):
    """The tuning hook takes up to eight K splits (the planner itself picks
    at most four): the finisher reads the other splits' slots four at a
    time. Against the FP64 oracle, and deterministic."""
    rng = np.random.default_rng([rows, cols, batch, *plan])
    m = _matrix(rng, rows, cols, 4, 64, kind)
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    want = oracle.matmul_f64(*m, kind, x, rows, cols, 4, 64, batch, 16)
    print(f"many splits {rows}x{cols} B={batch} plan {plan}", flush=True)
    got, kernel = _run(gpu, m, x, rows, cols, 4, 64, batch, kind, (-4, _ks(*plan)))
    ring, ns, tr, kw = plan
    assert kernel.removesuffix(" elect") == f"affine_band_kernel ring={ring} ns={ns} tr={tr} kw={kw}", kernel
    assert_gate(got, want, f"{rows}x{cols} B={batch} plan {plan} ({kernel})")
    again, _ = _run(gpu, m, x, rows, cols, 4, 64, batch, kind, (-4, _ks(*plan)))
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "launches differ"

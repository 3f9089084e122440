"""The fused forms on the GPU through the C ABI, against the FP64 oracle of
the reference's unfused sequence (src/engine.rs:748-765):

  rms_norm -> gate.matvec, up.matvec -> swiglu   ==  mlp_gate_up_swiglu[_bf16|_f16meta]
  down.matvec -> add                             ==  matmul_affine_add[_bf16|_f16meta]

Both are additions with no reference counterpart; the gate is the one the
unfused products meet (rel-L2 <= 1e-5, max-abs <= 1e-4 * max|y64|).
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


def _up(gpu, m):
    return [gpu.upload_bytes(np.ascontiguousarray(a)) for a in m]


def _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, bits, group, batch, kind):
    bufs = _up(gpu, gate_m) + _up(gpu, up_m) + [gpu.upload_f32(x.ravel()), gpu.upload_f32(nw),
                                                gpu.alloc_f32(batch * rows)]
    gpu.dispatch("mlp_gate_up_swiglu" + SUFFIX[kind], bufs, [rows, cols, bits, group, batch, EPS_BITS])
    return gpu.read_f32(bufs[-1], batch * rows)


@pytest.mark.parametrize("rows,cols,bits,group,batch,kind", [
    (17408, 5120, 4, 64, 1, "bf16"),   # the 27B MLP's gate/up at decode
    (17408, 5120, 4, 64, 3, "bf16"),   # the MTP verification block
    (300, 512, 4, 32, 2, "f32"),       # row tail, FP32 metadata
    (1000, 1024, 8, 64, 1, "f16"),     # Q8, F16 metadata
    (64, 2048, 4, 128, 4, "bf16"),     # group 128, four RHS
    (24, 4096, 8, 32, 2, "bf16"),      # fewer rows than one tile pair
])
@pytest.mark.parametrize("rr", [0, -2, -3])
def test_mlp_gate_up_swiglu_matches_unfused_oracle(gpu, rr, rows, cols, bits, group, batch, kind):
    """Default plan (the row-band kernel's MLP form where it has a one-round
    plan for both matrices' grid), the split-K kernel forced (rr -2) and the
    row-owning kernel's MLP mode forced (rr -3)."""
    rng = np.random.default_rng(rows + 7 * cols + batch)
    gate_m = _matrix(rng, rows, cols, bits, group, kind)
    up_m = _matrix(rng, rows, cols, bits, group, kind)
    x = rng.standard_normal((batch, cols)).astype(np.float32) * 3
    nw = rng.uniform(0.2, 1.8, cols).astype(np.float32)
    want = oracle.mlp_gate_up_f64(gate_m, up_m, kind, x, nw, EPS, rows, cols, bits, group, batch, 8)
    gpu.set_gemv_plan(rr, 0)
    try:
        got = _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, bits, group, batch, kind)
        assert_gate(got, want, f"mlp {rows}x{cols} Q{bits}/g{group} {kind} B{batch} rr={rr}")
        again = _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, bits, group, batch, kind)
        assert np.array_equal(again.view(np.uint32), got.view(np.uint32)), "launches differ"
    finally:
        gpu.set_gemv_plan(0, 0)


@pytest.mark.parametrize("plan", [310201, 220401, 330402, 240801, 210204])
@pytest.mark.parametrize("rows,cols,bits,group,batch,kind", [
    (2000, 3072, 4, 64, 2, "bf16"), (1000, 1024, 8, 64, 1, "f16"), (300, 2048, 4, 32, 2, "f32")])
def test_mlp_band_form_forced_plans(gpu, plan, rows, cols, bits, group, batch, kind):
    """The row-band kernel's MLP form under forced plans (rr -4, ks = ring *
    100000 + splits * 10000 + tiles * 100 + waves): one to four K splits
    (the gate and up slot planes), bands of one to four gate tiles with as
    many up tiles, one to four waves per tile, row tails; against the FP64
    oracle and deterministic."""
    rng = np.random.default_rng(plan % 9973 + rows + batch)
    gate_m = _matrix(rng, rows, cols, bits, group, kind)
    up_m = _matrix(rng, rows, cols, bits, group, kind)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    want = oracle.mlp_gate_up_f64(gate_m, up_m, kind, x, nw, EPS, rows, cols, bits, group, batch, 8)
    gpu.set_gemv_plan(-4, plan)
    try:
        got = _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, bits, group, batch, kind)
        kernel = gpu.last_hip_kernel()
        again = _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, bits, group, batch, kind)
    finally:
        gpu.set_gemv_plan(0, 0)
    ring, ns, tr, kw = plan // 100000, plan // 10000 % 10, plan // 100 % 100, plan % 100
    assert kernel == f"affine_band_kernel ring={ring} ns={ns} tr={tr} kw={kw} (MLP)", kernel
    assert_gate(got, want, f"mlp band {plan} {rows}x{cols} Q{bits}/g{group} {kind} B{batch}")
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "launches differ"


@pytest.mark.parametrize("plan,batch", [(320801, 3), (220401, 2), (340401, 4)])
def test_mlp_band_form_with_elected_finishers(gpu, plan, batch):
    """The row-band MLP form at the 27B gate/up shape under forced split
    plans whose workgroups take several rounds: every split publishes its
    gate, up and sum-of-squares slots, and the band's last workgroup to
    arrive finishes. Against the FP64 oracle and deterministic."""
    rows, cols = 17408, 5120
    rng = np.random.default_rng(plan + batch)
    gate_m = _matrix(rng, rows, cols, 4, 64, "bf16")
    up_m = _matrix(rng, rows, cols, 4, 64, "bf16")
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    want = oracle.mlp_gate_up_f64(gate_m, up_m, "bf16", x, nw, EPS, rows, cols, 4, 64, batch, 16)
    print(f"mlp elected plan {plan} B={batch}", flush=True)
    gpu.set_gemv_plan(-4, plan)
    try:
        got = _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, 4, 64, batch, "bf16")
        kernel = gpu.last_hip_kernel()
        again = _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, 4, 64, batch, "bf16")
    finally:
        gpu.set_gemv_plan(0, 0)
    ring, ns, tr, kw = plan // 100000, plan // 10000 % 10, plan // 100 % 100, plan % 100
    assert kernel == f"affine_band_kernel ring={ring} ns={ns} tr={tr} kw={kw} elect (MLP)", kernel
    assert_gate(got, want, f"mlp elected {plan} B{batch}")
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "launches differ"


@pytest.mark.parametrize("batch", [1, 2, 3, 4])
def test_mlp_default_is_the_band_kernel_at_the_27b_shape(gpu, batch):
    """At the 27B gate/up shape the fused form runs on the row-band kernel:
    each band holds gate tiles and the up tiles of the same rows, so one
    staging of x serves both matrices and the grid is one matrix's. At B=1
    a plan fits one round of resident workgroups; at B=2 and B=3 none does,
    and single-split bands of two gate and two up tiles run over several
    rounds with x staged in two phases; at B=4, 8-tile bands in two splits
    with elected finishers."""
    rows, cols = 17408, 5120
    rng = np.random.default_rng(batch)
    gate_m = _matrix(rng, rows, cols, 4, 64, "bf16")
    up_m = _matrix(rng, rows, cols, 4, 64, "bf16")
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, 4, 64, batch, "bf16")
    kernel = gpu.last_hip_kernel()
    want = {1: "affine_band_kernel ring=2 ns=1 tr=4 kw=1 (MLP)",
            2: "affine_band_kernel ring=2 ns=1 tr=4 kw=1 phased (MLP)",
            3: "affine_band_kernel ring=2 ns=1 tr=4 kw=1 phased (MLP)",
            4: "affine_band_kernel ring=2 ns=2 tr=8 kw=1 elect (MLP)"}[batch]
    assert kernel == want, kernel


@pytest.mark.parametrize("plan,batch", [(0, 2), (0, 3), (0, 4), (2210401, 2), (2310401, 3), (2210401, 1)])
def test_mlp_band_form_single_split_over_several_rounds(gpu, plan, batch):
    """The row-band MLP form at the 27B gate/up shape with single-split
    bands over several rounds of workgroups (the default at B=2..4, and
    forced plans with x staged in two phases: the norm weights and the sums
    of squares of the second half's columns are taken when that half is
    staged). Against the FP64 oracle and deterministic."""
    rows, cols = 17408, 5120
    rng = np.random.default_rng(plan + batch + 3)
    gate_m = _matrix(rng, rows, cols, 4, 64, "bf16")
    up_m = _matrix(rng, rows, cols, 4, 64, "bf16")
    x = rng.standard_normal((batch, cols)).astype(np.float32) * 3
    nw = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    want = oracle.mlp_gate_up_f64(gate_m, up_m, "bf16", x, nw, EPS, rows, cols, 4, 64, batch, 16)
    print(f"mlp single-split plan {plan} B={batch}", flush=True)
    gpu.set_gemv_plan(-4 if plan else 0, plan)
    try:
        got = _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, 4, 64, batch, "bf16")
        kernel = gpu.last_hip_kernel()
        again = _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, 4, 64, batch, "bf16")
    finally:
        gpu.set_gemv_plan(0, 0)
    assert kernel.startswith("affine_band_kernel") and kernel.endswith("(MLP)"), kernel
    if plan:
        assert kernel.endswith(" ns=1 tr=4 kw=1 phased (MLP)"), kernel
    assert_gate(got, want, f"mlp single-split {plan} B{batch} ({kernel})")
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "launches differ"


def test_mlp_rms_statistic_covers_every_column_and_rhs(gpu):
    """The norm's statistic is per RHS over all columns: scaling one RHS's x
    leaves its output unchanged (up to eps) and does not touch the others."""
    rows, cols, batch = 64, 4096, 3
    rng = np.random.default_rng(5)
    gate_m = _matrix(rng, rows, cols, 4, 64, "bf16")
    up_m = _matrix(rng, rows, cols, 4, 64, "bf16")
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    nw = np.ones(cols, np.float32)
    base = _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, 4, 64, batch, "bf16").reshape(batch, rows)
    x2 = x.copy()
    x2[1] *= 64.0  # exact in FP32
    got = _run_mlp(gpu, gate_m, up_m, x2, nw, rows, cols, 4, 64, batch, "bf16").reshape(batch, rows)
    assert np.array_equal(got[0], base[0]) and np.array_equal(got[2], base[2])
    np.testing.assert_allclose(got[1], base[1], rtol=2e-4, atol=1e-5 * np.abs(base[1]).max())


def _run_add(gpu, m, x, r, rows, cols, bits, group, batch, kind, in_place):
    w, s, b = _up(gpu, m)
    xb = gpu.upload_f32(x.ravel())
    rb = gpu.upload_f32(r.ravel())
    yb = rb if in_place else gpu.alloc_f32(batch * rows)
    gpu.dispatch("matmul_affine_add" + SUFFIX[kind], [w, s, b, xb, rb, yb], [rows, cols, bits, group, batch])
    return gpu.read_f32(yb, batch * rows), gpu.read_f32(rb, batch * rows)


@pytest.mark.parametrize("rr", [0, -2, -3])
@pytest.mark.parametrize("rows,cols,bits,group,batch,kind", [
    (5120, 17408, 4, 64, 1, "bf16"),   # the 27B MLP's down projection
    (5120, 17408, 4, 64, 3, "bf16"),
    (300, 4096, 8, 32, 2, "f16"),
    (151936 // 8, 5120, 4, 64, 1, "f32"),
])
def test_matmul_affine_add_matches_product_plus_residual(gpu, rr, rows, cols, bits, group, batch, kind):
    """y = r + W x on every matrix-core kernel (default plan, split-K forced,
    row-owning forced), in place (y is r's view) and into a separate y."""
    rng = np.random.default_rng(rows + cols + batch + rr)
    m = _matrix(rng, rows, cols, bits, group, kind)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    r = rng.standard_normal((batch, rows)).astype(np.float32) * 10
    want = oracle.matmul_add_f64(*m, kind, x, r, rows, cols, bits, group, batch, 8)
    gpu.set_gemv_plan(rr, 0)
    try:
        got, r_after = _run_add(gpu, m, x, r, rows, cols, bits, group, batch, kind, in_place=False)
        assert np.array_equal(r_after, r.ravel()), "the residual input was modified"
        assert_gate(got, want, f"add {rows}x{cols} {kind} B{batch} rr={rr}")
        got2, r2 = _run_add(gpu, m, x, r, rows, cols, bits, group, batch, kind, in_place=True)
        assert np.array_equal(got2.view(np.uint32), got.view(np.uint32)), "in-place result differs"
    finally:
        gpu.set_gemv_plan(0, 0)


def test_residual_form_on_a_matrix_too_tall_for_one_round(gpu):
    """y = r + W x where no row-band plan fits one round of resident
    workgroups (about 1563 bands of 8 tiles): single-split bands over
    several rounds, with a partial last tile and band, in place and into a
    separate y, against the FP64 oracle."""
    rows, cols, batch = 200003, 1024, 2
    rng = np.random.default_rng(11)
    m = _matrix(rng, rows, cols, 4, 64, "bf16")
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    r = rng.standard_normal((batch, rows)).astype(np.float32) * 10
    want = oracle.matmul_add_f64(*m, "bf16", x, r, rows, cols, 4, 64, batch, 8)
    gpu.set_gemv_plan(0, 0)
    got, r_after = _run_add(gpu, m, x, r, rows, cols, 4, 64, batch, "bf16", in_place=False)
    kernel = gpu.last_hip_kernel()
    assert kernel.startswith("affine_band_kernel ring=") and \
        kernel.removesuffix(" phased").endswith(" ns=1 tr=8 kw=1"), kernel
    assert np.array_equal(r_after, r.ravel()), "the residual input was modified"
    assert_gate(got, want, f"add {rows}x{cols} B{batch} multi-round")
    got2, _ = _run_add(gpu, m, x, r, rows, cols, 4, 64, batch, "bf16", in_place=True)
    assert np.array_equal(got2.view(np.uint32), got.view(np.uint32)), "in-place result differs"


def test_fused_alias_rules_and_reference_mode(gpu):
    rows, cols = 64, 512
    rng = np.random.default_rng(1)
    w, s, b = _up(gpu, _matrix(rng, rows, cols, 4, 64, "bf16"))
    x = gpu.upload_f32(rng.standard_normal(cols).astype(np.float32))
    big = gpu.upload_f32(np.zeros(2 * rows, np.float32))
    params = [rows, cols, 4, 64, 1]
    # y overlapping r without being the same view, and y over x, are rejected.
    with pytest.raises(qmr.QmrError, match="output overlaps input buffer 4"):
        gpu.dispatch("matmul_affine_add_bf16", [w, s, b, x, big, big], params, offsets=[0, 0, 0, 0, 0, 4])
    with pytest.raises(qmr.QmrError, match="output overlaps input buffer 3"):
        gpu.dispatch("matmul_affine_add_bf16", [w, s, b, x, big, x], params)
    nw = gpu.upload_f32(np.ones(cols, np.float32))
    with pytest.raises(qmr.QmrError, match="output overlaps input buffer 7"):
        gpu.dispatch("mlp_gate_up_swiglu_bf16", [w, s, b, w, s, b, x, nw, nw], params + [EPS_BITS])
    # Group 32 holds at most two RHS in the matrix-core tile: no fused kernel.
    with pytest.raises(qmr.QmrError, match="no fused kernel for this format"):
        w32, s32, b32 = _up(gpu, _matrix(rng, rows, cols, 4, 32, "bf16"))
        x3 = gpu.upload_f32(np.ones(3 * cols, np.float32))
        gpu.dispatch("mlp_gate_up_swiglu_bf16", [w32, s32, b32, w32, s32, b32, x3, nw, gpu.alloc_f32(3 * rows)],
                     [rows, cols, 4, 32, 3, EPS_BITS])
    ref = qmr.Gpu("aligned", reference=True)
    try:
        rw, rs, rb = _up(ref, _matrix(rng, rows, cols, 4, 64, "f32"))
        rx, ry = ref.upload_f32(np.ones(cols, np.float32)), ref.alloc_f32(rows)
        # A residual product is a block: the block ban fires first.
        with pytest.raises(qmr.QmrError, match="dispatch is unavailable in reference mode"):
            ref.dispatch("matmul_affine_add", [rw, rs, rb, rx, ry, ry], params)
        rn = ref.upload_f32(np.ones(cols, np.float32))
        with pytest.raises(qmr.QmrError, match="Fused dispatch is unavailable in reference mode"):
            ref.dispatch("mlp_gate_up_swiglu", [rw, rs, rb, rw, rs, rb, rx, rn, ref.alloc_f32(rows)],
                         params + [EPS_BITS])
    finally:
        ref.close()


@pytest.mark.parametrize("rows,cols,bits,group,batch,kind,ring,tr", [
    (2000, 3072, 4, 64, 2, "bf16", 2, 4),    # 12 entries: the second phase from entry 6
    (1000, 1024, 8, 64, 1, "f16", 3, 2),     # Q8, F16 metadata, 8 entries: phases of 3 and 5
    (300, 2048, 4, 128, 3, "f32", 2, 4),     # group 128, FP32 metadata, row tail
    (130, 4160, 4, 64, 4, "bf16", 3, 8),     # K ends inside a tile and an entry, four RHS
])
def test_mlp_band_form_two_phase_staging_forced(gpu, rows, cols, bits, group, batch, kind, ring, tr):
    """The MLP form with x staged in two phases, forced (ks = 2000000 +
    ring*100000 + 10000 + tr*100 + 1) over formats and tails: the second
    phase loads its columns' x and norm weights and adds their x² to each
    RHS's statistic before the SwiGLU. Against the FP64 oracle, and
    deterministic."""
    rng = np.random.default_rng([rows, cols, bits, group, batch, 5])
    gate_m = _matrix(rng, rows, cols, bits, group, kind)
    up_m = _matrix(rng, rows, cols, bits, group, kind)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    want = oracle.mlp_gate_up_f64(gate_m, up_m, kind, x, nw, EPS, rows, cols, bits, group, batch, 8)
    plan = 2000000 + ring * 100000 + 10000 + tr * 100 + 1
    print(f"mlp two-phase {rows}x{cols} Q{bits}/g{group} {kind} B={batch} plan {plan}", flush=True)
    gpu.set_gemv_plan(-4, plan)
    try:
        got = _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, bits, group, batch, kind)
        kernel = gpu.last_hip_kernel()
        again = _run_mlp(gpu, gate_m, up_m, x, nw, rows, cols, bits, group, batch, kind)
    finally:
        gpu.set_gemv_plan(0, 0)
    assert kernel == f"affine_band_kernel ring={ring} ns=1 tr={tr} kw=1 phased (MLP)", kernel
    assert_gate(got, want, f"mlp two-phase {plan} {rows}x{cols} Q{bits}/g{group} {kind} B{batch}")
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "launches differ"

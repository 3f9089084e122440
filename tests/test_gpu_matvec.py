"""GEMV parity on the GPU through the C ABI against the FP64 oracle.

Restates the reference's GPU tests of its matvec pipelines:
  src/gpu.rs:1637-1732            known answers (Q4 nibbles, Q8, dense, embeddings)
  tests/quantized.rs:7-85         Q4/Q8 x groups x column/row tails x modes
  tests/bf16_metadata.rs:7-99     the same grid with BF16 metadata + embeddings
and adds the F16-metadata names, every compiled tiling of the GEMV kernel,
and BASELINE config 0 against its committed golden vector.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle
import qmr
import qmr.synth as synth
from helpers import (assert_close_ref, assert_gate, reference_metadata, reference_x, rotl,
                     run_affine, to_bf16_truncated, xorshift_words)

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def test_affine_q4_little_nibbles_and_bias(gpus):
    # src/gpu.rs:1637-1657
    for mode, gpu in gpus.items():
        w = gpu.upload_bytes(np.array([0x76543210, 0xFEDCBA98], np.uint32))
        s = gpu.upload_f32([2.0, 0.5])
        b = gpu.upload_f32([-1.0, -4.0])
        x = gpu.upload_f32(np.ones(8))
        y = gpu.alloc_f32(2)
        cmd = gpu.begin()
        cmd.encode("matvec_affine", [w, s, b, x, y], [2, 8, 4, 8], 64, 128)
        cmd.finish()
        assert gpu.read_f32(y, 2).tolist() == [48.0, 14.0], mode


def test_dense_and_q8_matvec_and_embedding(gpu):
    # src/gpu.rs:1699-1732
    dense = np.array([1, 2, 3, 4, -1, 0, 1, 2], np.float16).view(np.uint16)
    w = gpu.upload_bytes(dense)
    x = gpu.upload_f32([1, 2, 3, 4])
    y = gpu.alloc_f32(2)
    gpu.dispatch("matvec_f16", [w, x, y], [2, 4])
    np.testing.assert_allclose(gpu.read_f32(y, 2), [30, 10], rtol=3e-5)
    emb = gpu.alloc_f32(4)
    gpu.dispatch("embed_f16", [w, emb], [1, 4])
    assert gpu.read_f32(emb, 4).tolist() == [-1, 0, 1, 2]
    q = gpu.upload_bytes(np.array([0xFF800100, 0x04030201], np.uint32))
    s = gpu.upload_f32([0.5, 2.0])
    b = gpu.upload_f32([-1.0, -3.0])
    gpu.dispatch("matvec_affine", [q, s, b, x, y], [2, 4, 8, 4])
    np.testing.assert_allclose(gpu.read_f32(y, 2), [693, 30], rtol=3e-5)
    gpu.dispatch("embed_affine", [q, s, b, emb], [0, 4, 8, 4])
    assert gpu.read_f32(emb, 4).tolist() == [-1.0, -0.5, 63.0, 126.5]


def _quantized_case(bits, group, cols, rows):
    pack = 32 // bits
    seed = 0x84213957 ^ bits ^ rotl(group, 7) ^ rotl(cols, 13) ^ rotl(rows, 19)
    w = xorshift_words(seed, rows * cols // pack)
    s, b = reference_metadata(rows * cols // group)
    return w, s, b, reference_x(cols)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_specialized_q4_q8_match_scalar_across_groups_and_row_tails(gpus, bits, group):
    # tests/quantized.rs:7-85: every mode, tolerance 2e-4 + 2e-5*|want|.
    for cols in (group, 3 * group, 5120):
        for rows in (1, 3, 7, 19, 20):
            w, s, b, x = _quantized_case(bits, group, cols, rows)
            want = oracle.matmul_f64(w, s, b, "f32", x, rows, cols, bits, group)
            for mode, gpu in gpus.items():
                got = run_affine(gpu, "matvec_affine", w, s, b, x, rows, cols, bits, group)
                assert_close_ref(got, want, 2e-4, 2e-5, f"{mode} Q{bits}/g{group} {rows}x{cols}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("meta", ["bf16", "f16"])
def test_16bit_metadata_matches_scalar_for_groups_shapes_and_embeddings(gpus, bits, group, meta):
    # tests/bf16_metadata.rs:7-99, plus the same grid with F16 metadata.
    name = "matvec_affine_bf16" if meta == "bf16" else "matvec_affine_f16meta"
    embed = "embed_affine_bf16" if meta == "bf16" else "embed_affine_f16meta"
    for cols in (group, 3 * group, 5120):
        for rows in (1, 3, 7, 19, 20):
            pack = 32 // bits
            w = xorshift_words(0x1478ABCF, rows * cols // pack)
            s, b = reference_metadata(rows * cols // group)
            if meta == "bf16":
                s16, b16 = to_bf16_truncated(s), to_bf16_truncated(b)
            else:
                s16, b16 = s.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
            x = reference_x(cols)
            want = oracle.matmul_f64(w, s16, b16, meta, x, rows, cols, bits, group)
            for mode in ("aligned", "packed4", "stream"):
                gpu = gpus[mode]
                got = run_affine(gpu, name, w, s16, b16, x, rows, cols, bits, group)
                assert_close_ref(got, want, 2e-4, 2e-5, f"{mode} {name} Q{bits}/g{group} {rows}x{cols}")
            gpu = gpus["aligned"]
            wb, sb, bb = (gpu.upload_bytes(a) for a in (w, s16, b16))
            eb = gpu.alloc_f32(cols)
            gpu.dispatch(embed, [wb, sb, bb, eb], [rows - 1, cols, bits, group])
            got = gpu.read_f32(eb, cols)
            exact = oracle.dequant_row(w, s16, b16, meta, rows - 1, cols, bits, group)
            assert np.array_equal(got.view(np.uint32), exact.view(np.uint32)), "embedding bits"


def test_bf16_dispatch_is_unavailable_in_reference_mode(gpus):
    gpu = gpus["reference"]
    w = gpu.upload_bytes(np.zeros(64, np.uint32))
    m = gpu.upload_bytes(np.zeros(8, np.uint16))
    x = gpu.upload_f32(np.zeros(512))
    y = gpu.alloc_f32(1)
    with pytest.raises(qmr.QmrError, match="reference mode"):
        gpu.dispatch("matvec_affine_bf16", [w, m, m, x, y], [1, 512, 4, 64])
    with pytest.raises(qmr.QmrError, match="reference mode"):
        gpu.dispatch("matmul_affine", [w, m, m, x, y], [1, 512, 4, 64, 1])


# (-3, rt*100 + kw): row-owning matrix-core kernel with a pinned workgroup
# shape (0 = its planner); (-2, 0): split-K matrix-core kernel; the rest are
# the vector-ALU tilings.
PLANS = [(-3, 0), (-3, 102), (-3, 104), (-3, 116), (-3, 204), (-3, 208), (-3, 402), (-3, 801),
         (-2, 0), (-1, 0), (1, 1), (2, 1), (4, 1), (5, 2), (2, 2)]


@pytest.mark.parametrize("rr,ks", PLANS)
def test_every_compiled_tiling_matches_oracle(gpu, rr, ks):
    """Each (rows-per-slot, K-split) instance, with row tails (rows not a
    multiple of the tile), column tails (a partial round of chunks), both
    code widths, the three metadata types and batches 1..4."""
    gpu.set_gemv_plan(rr, ks)
    try:
        rng = np.random.default_rng(abs(rr) * 10 + ks % 97 + (rr < 0))
        for bits, meta, rows, cols in [(4, "bf16", 37, 1536), (4, "f32", 41, 64 * 17),
                                       (8, "f16", 23, 1024 + 256), (4, "f16", 3, 5120),
                                       (8, "bf16", 45, 64 * 9)]:
            group = 64
            pack = 32 // bits
            w = rng.integers(0, 2**32, rows * cols // pack, dtype=np.uint32)
            sf = rng.uniform(0.002, 0.02, rows * cols // group).astype(np.float32)
            bf = (-(2 ** (bits - 1)) * sf + rng.normal(0, 1e-3, sf.size)).astype(np.float32)
            if meta == "bf16":
                s, b = synth.f32_to_bf16_bits(sf), synth.f32_to_bf16_bits(bf)
            elif meta == "f16":
                s, b = sf.astype(np.float16).view(np.uint16), bf.astype(np.float16).view(np.uint16)
            else:
                s, b = sf, bf
            suffix = {"bf16": "_bf16", "f16": "_f16meta", "f32": ""}[meta]
            for batch in (1, 2, 3, 4):
                x = rng.standard_normal((batch, cols)).astype(np.float32)
                want = oracle.matmul_f64(w, s, b, meta, x, rows, cols, bits, group, batch)
                got = run_affine(gpu, "matmul_affine" + suffix, w, s, b, x, rows, cols, bits,
                                 group, batch)
                assert_gate(got, want, f"plan {rr},{ks} Q{bits} {meta} {rows}x{cols} B{batch}")
    finally:
        gpu.set_gemv_plan(0, 0)


def test_config0_golden_meets_gate(gpu):
    z = np.load(GOLDEN / "config0.npz")
    seed = int(z["seed"])
    m = synth.q4_bf16_matrix(1024, 1024, seed, tag="config0")
    x = synth.activations(1024, 1, seed, tag="config0")
    assert np.array_equal(m.w[:16], z["w_head"])
    got = run_affine(gpu, "matvec_affine_bf16", m.w, m.s, m.b, x, 1024, 1024, 4, 64)
    assert gpu.last_kernel() == "matvec_q4_g64_aligned_bf16"
    assert_gate(got, z["y64"], "config 0")


SPLIT_SHAPES = [(5120, 17408, 1), (37, 64 * 136, 3), (300, 4096, 2), (64, 32 * 128, 4),
                (1000, 64 * 30, 1)]


def _launch_three(gpu, rows, cols, batch, seed):
    """Three launches of one product in one command (distinct outputs)."""
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 2**32, rows * cols // 8, dtype=np.uint32)
    sf = rng.uniform(0.002, 0.02, rows * cols // 64).astype(np.float32)
    bf = (-8 * sf + rng.normal(0, 1e-3, sf.size)).astype(np.float32)
    s, b = synth.f32_to_bf16_bits(sf), synth.f32_to_bf16_bits(bf)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    wb, sb, bb = gpu.upload_bytes(w), gpu.upload_bytes(s), gpu.upload_bytes(b)
    xb = gpu.upload_f32(x.ravel())
    ys = [gpu.alloc_f32(batch * rows) for _ in range(3)]
    params = [rows, cols, 4, 64, batch]
    _, threads = qmr.dispatch_layout("matmul_affine_bf16", params)
    cmd = gpu.begin()
    for yb in ys:
        cmd.encode("matmul_affine_bf16", [wb, sb, bb, xb, yb], params, threads, 128)
    cmd.finish()
    cmd.release()
    got = [gpu.read_f32(yb, batch * rows) for yb in ys]
    want = oracle.matmul_f64(w, s, b, "bf16", x, rows, cols, 4, 64, batch, 8)
    return got, want


@pytest.mark.parametrize("rows,cols,batch", SPLIT_SHAPES)
def test_split_k_reduction_is_deterministic_across_launches(gpu, rows, cols, batch):
    """The split-K matrix-core kernel's reduction (the last workgroup of a
    band to arrive adds the partials in split order): several launches in one
    command give bit-identical y that meets the gate; row tails included."""
    gpu.set_gemv_plan(-2, 0)
    try:
        plan = gpu.gemv_plan(rows, cols, 4, batch)
        assert plan[0] == -2 and plan[1] > 1, f"expected a split-K matrix-core plan, got {plan}"
        got, want = _launch_three(gpu, rows, cols, batch, rows * 7 + batch)
    finally:
        gpu.set_gemv_plan(0, 0)
    for g in got[1:]:
        assert np.array_equal(g.view(np.uint32), got[0].view(np.uint32)), "launches differ"
    assert_gate(got[0], want, f"split-K {plan} {rows}x{cols} B{batch}")


@pytest.mark.parametrize("rows,cols,batch", SPLIT_SHAPES)
def test_row_kernel_is_deterministic(gpu, rows, cols, batch):
    """The row-owning matrix-core kernel (opt-in) under its own planner:
    repeated launches give bit-identical y that meets the gate."""
    gpu.set_gemv_plan(-3, 0)
    try:
        plan = gpu.gemv_plan(rows, cols, 4, batch)
        assert plan[0] == -3, f"expected the row-owning kernel, got {plan}"
        got, want = _launch_three(gpu, rows, cols, batch, rows * 11 + batch)
    finally:
        gpu.set_gemv_plan(0, 0)
    for g in got[1:]:
        assert np.array_equal(g.view(np.uint32), got[0].view(np.uint32)), "launches differ"
    assert_gate(got[0], want, f"rows {plan} {rows}x{cols} B{batch}")


@pytest.mark.parametrize("rows,cols,bits,batch,kind", [
    (5120, 17408, 4, 1, -4), (17408, 5120, 4, 3, -4), (5120, 5120, 4, 1, -4), (5120, 17408, 8, 1, -4),
    (5120, 5120, 8, 3, -4), (5120, 5120, 4, 3, -4), (151936, 5120, 4, 1, -4), (151936, 5120, 4, 3, -4)])
def test_default_plan_kernel_family(gpu, rows, cols, bits, batch, kind):
    """The default planner takes the row-band kernel: a plan whose
    workgroups are all resident in one round where one exists (the Q4 and
    Q8 MLP shapes, 5120x5120 projections), else single-split bands over
    several rounds (the vocabulary head: 8 tiles per band, one wave per
    tile, the two-entry ring, two workgroups per CU: at B=3 with x staged
    in two phases, which makes room for the second workgroup)."""
    gpu.set_gemv_plan(0, 0)
    plan = gpu.gemv_plan(rows, cols, bits, batch)
    assert plan[0] == kind, f"{rows}x{cols} B{batch}: expected plan kind {kind}, got {plan}"
    if rows == 151936:
        assert plan[1] == (210801 if batch == 1 else 2210801), plan
    if rows == cols == 5120:
        # Short streams (under 8 entries per wave) at one RHS, and with 8-bit
        # codes, take half-height bands; Q4 at three RHS keeps the planner's
        # own pick.
        assert plan[1] // 100 % 100 == (2 if batch == 1 or bits == 8 else 4), plan
        # Streams of at most four entries per wave (Q4 here: 20 entries per
        # row over three splits of two waves) take the two-entry ring.
        assert plan[1] // 100000 % 10 == (2 if bits == 4 else 3), plan


@pytest.mark.parametrize("rr,name,batch", [(0, "matmul_affine_bf16", 1), (0, "matmul_affine_bf16", 3),
                                           (-2, "matmul_affine_bf16", 2), (-3, "matmul_affine_bf16", 2),
                                           (0, "matmul_affine_wide_bf16", 100)])
def test_matrix_core_kernels_read_x_at_4_byte_offsets(gpu, rr, name, batch):
    """x (and y) views 4-byte but not 16-byte aligned, as the block contract
    allows (tests/batch_matrix.rs:176-191; the BF16 matvec names require
    16-byte aligned input instead), with codes and metadata aligned so the
    matrix-core kernels (row-band, split-K, row-owning, wide) take the
    product: their x loads are 128-bit loads that need only 4-byte
    alignment."""
    rows, cols = 300, 4096
    rng = np.random.default_rng(batch * 7 + (rr < 0))
    w = rng.integers(0, 2**32, rows * cols // 8, dtype=np.uint32)
    sf = rng.uniform(0.002, 0.02, rows * cols // 64).astype(np.float32)
    bf = (-8 * sf + rng.normal(0, 1e-3, sf.size)).astype(np.float32)
    s, b = synth.f32_to_bf16_bits(sf), synth.f32_to_bf16_bits(bf)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    want = oracle.matmul_f64(w, s, b, "bf16", x, rows, cols, 4, 64, batch)
    gpu.set_gemv_plan(rr, 0)
    try:
        if batch <= 4:
            plan = gpu.gemv_plan(rows, cols, 4, batch)
            assert plan[0] in (-2, -3, -4), f"expected a matrix-core plan, got {plan}"
        wb, sb, bb = gpu.upload_bytes(w), gpu.upload_bytes(s), gpu.upload_bytes(b)
        xb = gpu.upload_f32(np.concatenate([[99.0], x.ravel()]).astype(np.float32))
        yb = gpu.upload_f32(np.full(batch * rows + 2, 12345.0, np.float32))
        params = [rows, cols, 4, 64] + ([batch] if name.startswith("matmul") else [])
        gpu.dispatch(name, [wb, sb, bb, xb, yb], params, offsets=[0, 0, 0, 4, 4])
        got = gpu.read_f32(yb, batch * rows + 2)
    finally:
        gpu.set_gemv_plan(0, 0)
    assert got[0] == 12345.0 and got[batch * rows + 1] == 12345.0
    assert_gate(got[1:batch * rows + 1], want, f"{name} B{batch} x at a 4-byte offset")


@pytest.mark.parametrize("plan", [(0, 0), (-1, 0)])
@pytest.mark.parametrize("rows,cols,batch", [
    (5120, 17408, 1), (17408, 5120, 3), (5120, 17408, 4), (301, 4104, 2), (4099, 2056, 3), (1000, 8, 4),
    (77, 1001, 1), (33, 512, 4)])
def test_dense_f16_products_at_scale(gpu, rows, cols, batch, plan):
    """matvec_f16 / matmul_f16 (kernels/qwen.metal:48-57,
    kernels/matmul_block.metal:213-248) against the FP64 oracle: the default
    choice (the matrix-core kernel for some products of 2-4 RHS), and with
    the rr = -1 hook the vector-ALU streaming kernel (cols % 8 == 0, any row
    tail, 1-4 RHS) in its three shapes (four waves splitting K over 4 or 8
    rows, one wave per 4 rows at 17408x5120 B=3; partial last steps and row
    groups); the simple kernel takes cols % 8 != 0 either way."""
    rng = np.random.default_rng(rows * 3 + cols + batch)
    w16 = rng.standard_normal(rows * cols).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    wb = gpu.upload_bytes(w16)
    xb = gpu.upload_f32(x.ravel())
    yb = gpu.upload_f32(np.full(batch * rows + 1, 7.0, np.float32))
    name = "matvec_f16" if batch == 1 else "matmul_f16"
    gpu.set_gemv_plan(*plan)
    try:
        gpu.dispatch(name, [wb, xb, yb], [rows, cols] + ([batch] if batch > 1 else []))
    finally:
        gpu.set_gemv_plan(0, 0)
    if plan == (-1, 0) or cols % 32 != 0:
        assert gpu.last_hip_kernel() == "dense_f16_kernel", gpu.last_hip_kernel()
    got = gpu.read_f32(yb, batch * rows + 1)
    assert got[-1] == 7.0, "wrote past y"
    want = oracle.dense_f16_f64(w16, x, rows, cols, batch)
    assert_gate(got[:-1], want, f"dense {rows}x{cols} B{batch}")


def test_forced_split_count_is_honoured_and_correct(gpu):
    """The tuning hook rr = -2, ks = n keeps only n K splits when feasible
    (17408x5120 at B=1: 10 splits), and the product still meets the gate;
    an infeasible count falls back to the split-K planner's own count."""
    rows, cols = synth.MLP_SHAPES["gate_up"]
    gpu.set_gemv_plan(-2, 0)
    try:
        split_k_default = gpu.gemv_plan(rows, cols, 4, 1)
        assert split_k_default[0] == -2
        gpu.set_gemv_plan(-2, 10)
        assert gpu.gemv_plan(rows, cols, 4, 1) == (-2, 10)
        got, want = _launch_three(gpu, rows, cols, 1, 41)
        assert_gate(got[0], want, "forced 10 splits")
        gpu.set_gemv_plan(-2, 31)
        assert gpu.gemv_plan(rows, cols, 4, 1) == split_k_default
    finally:
        gpu.set_gemv_plan(0, 0)


@pytest.mark.parametrize("sizes,offsets", [((44_564_480, 2_785_280, 2_785_280), (0, 0, 0, 0)),
                                           ((1_000_004, 36, 0), (4, 0, 0, 0)),
                                           ((20, 1_048_576, 4), (0, 8, 12, 4))])
def test_read_checksum_reads_every_word_once(gpu, sizes, offsets):
    """read_checksum (the read-floor kernel): the XOR of its slots equals the
    XOR of every 32-bit word of the three views, for word tails that are not
    16-byte multiples, an empty view and 4-byte view offsets."""
    rng = np.random.default_rng(sum(sizes))
    views = [rng.integers(0, 2**32, n // 4, dtype=np.uint64).astype(np.uint32) for n in sizes]
    bufs = []
    for v, off in zip(views, offsets[:3]):
        pad = np.full(off // 4, 0xDEADBEEF, np.uint32)
        bufs.append(gpu.upload_bytes(np.concatenate([pad, v, np.full(3, 0xABCDEF01, np.uint32)])))
    out = gpu.upload_bytes(np.full(4096 + offsets[3] // 4, 0x55555555, np.uint32))
    for launch in range(2):
        gpu.dispatch("read_checksum", bufs + [out], list(sizes), offsets=list(offsets))
        slots = np.frombuffer(out.read_bytes(offsets[3], 4096 * 4), np.uint32)
        want = np.uint32(0)
        for v in views:
            if v.size:
                want ^= np.bitwise_xor.reduce(v)
        assert np.bitwise_xor.reduce(slots) == want, f"launch {launch}"


def test_frame_gpu_seconds_is_device_time(gpu):
    """FrameTiming.gpu_seconds (src/gpu/timing.rs:8-21; the Metal command
    buffer's GPU start/end) covers the command's GPU work only: the start
    event is recorded right before the first launch, so host time spent
    between begin and the first encode is not counted. A wide block (two
    launches, ~0.1 ms) encoded after 50 ms of host sleep: gpu_seconds is at
    most the command's wall time and within 1.5x of the elapsed time between
    marks around the encode."""
    import time
    rng = np.random.default_rng(3)
    rows, cols, batch = 17408, 5120, 256
    w = rng.integers(0, 2**32, rows * cols // 8, dtype=np.uint64).astype(np.uint32)
    s = synth.f32_to_bf16_bits(rng.uniform(0.002, 0.02, rows * cols // 64).astype(np.float32))
    b = synth.f32_to_bf16_bits(rng.uniform(-0.1, 0.0, rows * cols // 64).astype(np.float32))
    x = rng.normal(0, 1, batch * cols).astype(np.float32)
    bufs = [gpu.upload_bytes(w), gpu.upload_bytes(s), gpu.upload_bytes(b), gpu.upload_f32(x),
            gpu.alloc_f32(batch * rows)]
    name, params = "matmul_affine_wide_bf16", [rows, cols, 4, 64, batch]
    _, threads = qmr.dispatch_layout(name, params)
    gpu.dispatch(name, bufs, params)  # workspace growth happens here, outside the timed command
    for _ in range(3):
        t0 = time.perf_counter()
        cmd = gpu.begin()
        time.sleep(0.05)
        a = cmd.mark()
        cmd.encode(name, bufs, params, threads, 128)
        c = cmd.mark()
        timing = cmd.finish()
        wall = time.perf_counter() - t0
        around = cmd.elapsed_ms(a, c) * 1e-3
        cmd.release()
        assert 0.0 < timing.gpu_seconds <= wall, (timing.gpu_seconds, wall)
        assert around / 1.5 <= timing.gpu_seconds <= around * 1.5, (timing.gpu_seconds, around)
    # A warm config-0 command (1024x1024 GEMV, a few microseconds): the marks
    # around it also hold the host's encode time, which the GPU time
    # excludes, so here only the upper bounds apply.
    m = synth.q4_bf16_matrix(1024, 1024, 1, tag="config0")
    x0 = synth.activations(1024, 1, 1, tag="config0")
    bufs0 = [gpu.upload_bytes(m.w), gpu.upload_bytes(m.s), gpu.upload_bytes(m.b), gpu.upload_f32(x0),
             gpu.alloc_f32(1024)]
    gpu.dispatch("matvec_affine_bf16", bufs0, [1024, 1024, 4, 64])
    for _ in range(3):
        t0 = time.perf_counter()
        cmd = gpu.begin()
        time.sleep(0.05)
        a = cmd.mark()
        cmd.encode("matvec_affine_bf16", bufs0, [1024, 1024, 4, 64], 1024 * 32, 128)
        c = cmd.mark()
        timing = cmd.finish()
        wall = time.perf_counter() - t0
        around = cmd.elapsed_ms(a, c) * 1e-3
        cmd.release()
        assert 0.0 < timing.gpu_seconds <= min(wall, around * 1.5), (timing.gpu_seconds, wall, around)


@pytest.mark.parametrize("name,bits,group", [("embed_affine", 4, 64), ("embed_affine", 8, 32),
                                             ("embed_affine_bf16", 4, 64), ("embed_affine_bf16", 8, 128),
                                             ("embed_f16", 0, 0)])
def test_embed_offset_writes_only_its_slot_bit_exact(gpu, name, bits, group):
    """Matrix::embed_offset (src/engine/block.rs:231-261): encode_offsets
    with the output view at byte offset slot*cols*4 of a [batch][cols]
    buffer, as the block path embeds token i into row i
    (src/engine/block.rs:426). The row lands bit-exact (RN32(q*s + b), or the
    F16 row widened) in its slot; every word before and after it keeps its
    guard value."""
    rng = np.random.default_rng([bits, group, len(name)])
    rows, cols, batch, slot, token = 9, 1024, 4, 2, 5
    guard = np.uint32(0x7FC0DEAD)  # a quiet NaN pattern no dequantised value has
    ybuf = gpu.upload_bytes(np.full(batch * cols, guard, np.uint32))
    if name == "embed_f16":
        dense = rng.normal(0, 1, rows * cols).astype(np.float16)
        bufs = [gpu.upload_bytes(dense.view(np.uint16))]
        params = [token, cols]
        want = dense.reshape(rows, cols)[token].astype(np.float32)
    else:
        w = rng.integers(0, 2**32, rows * cols * bits // 32, dtype=np.uint64).astype(np.uint32)
        s = rng.uniform(0.002, 0.02, rows * cols // group).astype(np.float32)
        b = rng.uniform(-0.2, 0.0, rows * cols // group).astype(np.float32)
        kind = "f32"
        if name.endswith("_bf16"):
            s, b, kind = synth.f32_to_bf16_bits(s), synth.f32_to_bf16_bits(b), "bf16"
        bufs = [gpu.upload_bytes(w), gpu.upload_bytes(s), gpu.upload_bytes(b)]
        params = [token, cols, bits, group]
        want = oracle.dequant_row(w, s, b, kind, token, cols, bits, group)
    offsets = [0] * len(bufs) + [slot * cols * 4]
    gpu.dispatch(name, bufs + [ybuf], params, offsets=offsets)
    got = np.frombuffer(ybuf.read_bytes(0, batch * cols * 4), np.uint32).reshape(batch, cols)
    assert np.array_equal(got[slot], want.view(np.uint32)), name
    others = np.delete(got, slot, axis=0)
    assert np.all(others == guard), name


def test_command_delay_holds_the_stream(gpu):
    """qmr_command_delay (a measurement aid with no reference counterpart)
    holds the device stream for the requested GPU time: marks around a
    300 us hold read at least that, and launches queued behind it run after
    it and stay correct. Requests above one second are rejected."""
    m = synth.q4_bf16_matrix(1024, 1024, 5, tag="config0")
    x = synth.activations(1024, 1, 5, tag="config0")
    bufs = [gpu.upload_bytes(m.w), gpu.upload_bytes(m.s), gpu.upload_bytes(m.b), gpu.upload_f32(x.ravel()),
            gpu.alloc_f32(1024)]
    _, threads = qmr.dispatch_layout("matvec_affine_bf16", [1024, 1024, 4, 64])
    cmd = gpu.begin()
    a = cmd.mark()
    cmd.delay(300)
    b = cmd.mark()
    cmd.encode("matvec_affine_bf16", bufs, [1024, 1024, 4, 64], threads, 128)
    cmd.finish()
    held = cmd.elapsed_ms(a, b)
    cmd.release()
    assert 0.29 <= held <= 50.0, held
    want = oracle.matmul_f64(m.w, m.s, m.b, "bf16", x, 1024, 1024, 4, 64)
    assert_gate(gpu.read_f32(bufs[4], 1024), want)
    cmd = gpu.begin()
    try:
        with pytest.raises(qmr.QmrError, match="at most 1000000"):
            cmd.delay(1_000_001)
    finally:
        cmd.finish()
        cmd.release()

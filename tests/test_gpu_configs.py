"""BASELINE configurations at full size on the GPU against the FP64 oracle,
with the BASELINE gate (rel-L2 <= 1e-5, max-abs <= 1e-4*max|y|), and bit-exact
dequantisation of sampled rows:
  1: Q4/g64 BF16 17408x5120 and 5120x17408, B=1
  2: the same matrices, B=3 (MTP verification block)
  3: Q8/g64 5120x5120 with F16 and with FP32 metadata; Q4/g64 BF16 head
     151936x5120 at B=1 and B=3 (every row against the oracle)
  4: wide block 17408x5120 x 128 and x 256 RHS (every row against the
     oracle)
"""
import os

import numpy as np
import pytest

import oracle
import qmr.synth as synth
from helpers import assert_gate, run_affine

pytestmark = pytest.mark.gpu
SEED = synth.DEFAULT_SEED
THREADS = min(16, os.cpu_count() or 1)
NAME = {"bf16": "_bf16", "f16": "_f16meta", "f32": ""}


def rows_subset(m: synth.PackedMatrix, rows):
    per_w = m.cols * m.bits // 32
    per_m = m.cols // m.group
    rows = np.asarray(rows)
    w = m.w.reshape(m.rows, per_w)[rows].ravel()
    s = m.s.reshape(m.rows, per_m)[rows].ravel()
    b = m.b.reshape(m.rows, per_m)[rows].ravel()
    return w, s, b


def check(gpu, m, batch, sample_rows=None, name=None):
    x = synth.activations(m.cols, batch, SEED, tag=f"cfg{m.rows}x{m.cols}")
    name = name or (("matvec_affine" if batch == 1 else "matmul_affine") + NAME[m.meta])
    got = run_affine(gpu, name, m.w, m.s, m.b, x, m.rows, m.cols, m.bits, m.group, batch)
    if sample_rows is None:
        want = oracle.matmul_f64(m.w, m.s, m.b, m.meta, x, m.rows, m.cols, m.bits, m.group, batch,
                                 THREADS)
        assert_gate(got, want, f"{synth.describe(m, batch)}")
    else:
        w, s, b = rows_subset(m, sample_rows)
        want = oracle.matmul_f64(w, s, b, m.meta, x, len(sample_rows), m.cols, m.bits, m.group,
                                 batch, THREADS)
        got_s = np.concatenate([got[t * m.rows + np.asarray(sample_rows)] for t in range(batch)])
        assert_gate(got_s, want, f"{synth.describe(m, batch)} sampled")
    return got


def check_dequant_rows(gpu, m, rows):
    wb, sb, bb = (gpu.upload_bytes(a) for a in (m.w, m.s, m.b))
    eb = gpu.alloc_f32(m.cols)
    for r in rows:
        gpu.dispatch("embed_affine" + NAME[m.meta], [wb, sb, bb, eb], [r, m.cols, m.bits, m.group])
        got = gpu.read_f32(eb, m.cols)
        want = oracle.dequant_row(m.w, m.s, m.b, m.meta, r, m.cols, m.bits, m.group)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"row {r}"


@pytest.mark.parametrize("shape", ["gate_up", "down"])
def test_config1_and_2_mlp_shapes(gpu, shape):
    rows, cols = synth.MLP_SHAPES[shape]
    m = synth.q4_bf16_matrix(rows, cols, SEED, tag=shape)
    check(gpu, m, 1)
    check(gpu, m, 3)
    check_dequant_rows(gpu, m, [0, 1, rows // 2, rows - 1])


def test_config3_q8_f16_and_f32_metadata(gpu):
    m = synth.q8_f16_matrix(*synth.Q8_SHAPE, SEED)
    check(gpu, m, 1)
    check(gpu, synth.to_f32_metadata(m), 1)
    check(gpu, m, 3)
    check_dequant_rows(gpu, m, [0, 4095, 5119])


def test_config3_vocabulary_head(gpu):
    rows, cols = synth.HEAD_SHAPE
    m = synth.q4_bf16_matrix(rows, cols, SEED, tag="head")
    check(gpu, m, 1)
    check(gpu, m, 3)
    check_dequant_rows(gpu, m, [0, rows - 1])


def test_multi_round_band_plan_on_a_ragged_tall_matrix(gpu):
    """A matrix too tall for any one-round row-band plan, with a partial
    last tile and band: single-split bands over several rounds of
    workgroups, against the oracle on sampled rows (the tail rows
    included), deterministic across launches."""
    rows, cols, batch = 140001, 4096, 2
    m = synth.q4_bf16_matrix(rows, cols, SEED, tag="tall")
    sample = sorted(set(list(range(0, rows, 89)) + [rows - 16, rows - 2, rows - 1]))
    gpu.set_gemv_plan(0, 0)
    first = check(gpu, m, batch, sample)
    kernel = gpu.last_hip_kernel()
    assert kernel.startswith("affine_band_kernel ring=") and \
        kernel.removesuffix(" phased").endswith(" ns=1 tr=8 kw=1"), kernel
    again = check(gpu, m, batch, sample)
    assert np.array_equal(first.view(np.uint32), again.view(np.uint32)), "launches differ"


@pytest.mark.parametrize("batch", [128, 256])
def test_config4_wide_block(gpu, batch):
    rows, cols = synth.MLP_SHAPES["gate_up"]
    m = synth.q4_bf16_matrix(rows, cols, SEED, tag="gate_up")
    print(f"config 4: {batch} RHS, every row against the oracle", flush=True)
    check(gpu, m, batch, name="matmul_affine_wide_bf16")


@pytest.mark.parametrize("rows,cols,batch,meta", [(300, 1024, 100, "bf16"), (128, 512, 64, "f32"),
                                                  (17, 512, 5, "bf16"), (1000, 2048, 256, "f32"),
                                                  (250, 1536, 65, "bf16"), (290, 4096, 40, "f32"),
                                                  (600, 6400, 33, "bf16"), (17000, 512, 128, "bf16"),
                                                  (300, 1024, 8, "bf16"), (300, 1024, 9, "f32"),
                                                  (64, 512, 1, "bf16")])
def test_wide_block_tails_and_metadata(gpu, rows, cols, batch, meta):
    """Wide blocks at ragged row and RHS counts, both wide names, against
    the FP64 oracle. The kernel's K quarters hold 16 groups at cols 4096 and
    25 at cols 6400, past one metadata chunk (12 groups for F32 metadata, 20
    for BF16), so those cases stage several chunks per wave; 17000 rows take
    the 272-row workgroups and a partial last row block."""
    rng = np.random.default_rng(rows + batch)
    w = rng.integers(0, 2**32, rows * cols // 8, dtype=np.uint32)
    sf = rng.uniform(0.002, 0.02, rows * cols // 64).astype(np.float32)
    bf = (-8 * sf + rng.normal(0, 1e-3, sf.size)).astype(np.float32)
    s, b = (synth.f32_to_bf16_bits(sf), synth.f32_to_bf16_bits(bf)) if meta == "bf16" else (sf, bf)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    name = "matmul_affine_wide" + NAME[meta]
    got = run_affine(gpu, name, w, s, b, x, rows, cols, 4, 64, batch)
    want = oracle.matmul_f64(w, s, b, meta, x, rows, cols, 4, 64, batch, THREADS)
    assert_gate(got, want, f"{name} {rows}x{cols} B{batch}")

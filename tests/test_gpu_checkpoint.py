"""Matrices loaded from MLX checkpoints straight into device buffers
(qmr_matrix_load, the reference's Matrix::load, src/engine.rs:48-135), then
multiplied on the GPU through the C ABI and checked against the FP64 oracle
on the same checkpoint's host arrays."""
from __future__ import annotations

import time
from pathlib import Path

import numpy as np
import pytest

import oracle
import qmr
import qmr.synth as synth
from helpers import assert_gate, write_config, write_tensor_file

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _fixture_checkpoint(d: Path, tag: str) -> list[tuple[str, int, int]]:
    """The reference's tiny-q4 (tag q4f16) or tiny-bf16 (q4bf16) matrices,
    from their extracted bytes, as one safetensors checkpoint."""
    z = np.load(GOLDEN / "mlx_fixtures.npz")
    keys = sorted({k.rsplit("/", 1)[0] for k in z.files if k.endswith("/shape")})
    tensors, out = [], []
    for key in keys:
        rows, cols = (int(v) for v in z[f"{key}/shape"])
        kind = z[f"{key}/{tag}/meta"].tobytes().decode()
        raw = "language_model." + key.replace("/", ".")
        tensors += [(raw + ".weight", "U32", [rows, cols // 8], z[f"{key}/{tag}/w"].tobytes()),
                    (raw + ".scales", kind, [rows, cols // 32], z[f"{key}/{tag}/s"].tobytes()),
                    (raw + ".biases", kind, [rows, cols // 32], z[f"{key}/{tag}/b"].tobytes())]
        out.append((key.replace("/", "."), rows, cols))
    write_config(d, quantization={"bits": 4, "group_size": 32, "mode": "affine"})
    write_tensor_file(d / "model.safetensors", tensors)
    return out


def _product(gpu: qmr.Gpu, m: qmr.Matrix, x: np.ndarray, batch: int) -> np.ndarray:
    suffix = "_bf16" if m.metadata_bf16 else ""
    name = ("matvec_affine" if batch == 1 else "matmul_affine") + suffix
    xb = gpu.upload_f32(x.ravel())
    yb = gpu.alloc_f32(batch * m.rows)
    params = [m.rows, m.cols, m.bits, m.group] + ([batch] if batch > 1 else [])
    gpu.dispatch(name, [m.weight, m.scales, m.biases, xb, yb], params)
    return gpu.read_f32(yb, batch * m.rows)


@pytest.mark.parametrize("tag,mode", [("q4bf16", "bf16"), ("q4bf16", "f32"), ("q4f16", "bf16"),
                                      ("q4f16", "f32")])
def test_fixture_matrices_load_and_multiply(tmp_path, tag, mode):
    """All 33 fixture matrices: the device holds the checkpoint's words
    unchanged and its metadata as BF16 exactly when the device's metadata
    mode is "bf16" and the values compact losslessly (the BF16 checkpoint
    always does, and the device's metadata_stats then report the reference's
    (33, 6576)); B=1 and B=3 products meet the gate."""
    names = _fixture_checkpoint(tmp_path, tag)
    gpu = qmr.Gpu("aligned", metadata=mode)
    try:
        with qmr.Checkpoint(tmp_path) as cp:
            for name, rows, cols in names:
                host = cp.matrix(name)
                m = cp.load(gpu, name, rows, cols)
                assert (m.rows, m.cols, m.bits, m.group) == (rows, cols, 4, 32)
                assert np.array_equal(m.weight.read(np.uint32, host.weights.size), host.weights), name
                if mode == "bf16" and tag == "q4bf16":
                    assert m.metadata_bf16, name
                if m.metadata_bf16:
                    got_s = (m.scales.read(np.uint16, host.scales.size).astype(np.uint32) << 16).view(np.float32)
                    got_b = (m.biases.read(np.uint16, host.biases.size).astype(np.uint32) << 16).view(np.float32)
                else:
                    got_s = m.scales.read(np.float32, host.scales.size)
                    got_b = m.biases.read(np.float32, host.biases.size)
                assert np.array_equal(got_s, host.scales) and np.array_equal(got_b, host.biases), name
                for batch in (1, 3):
                    x = np.random.default_rng(rows * 7 + batch).standard_normal((batch, cols)).astype(np.float32)
                    want = oracle.matmul_f64(host.weights, host.scales, host.biases, "f32", x, rows, cols, 4, 32,
                                             batch)
                    assert_gate(_product(gpu, m, x, batch), want, f"{name} {mode} B{batch}")
        if mode == "f32":
            assert gpu.metadata_stats()[0] == 0
        if (tag, mode) == ("q4bf16", "bf16"):
            # tests/bf16_inference.rs:11-15: every tiny-bf16 matrix compacted,
            # 3288 scales and biases kept at 2 bytes instead of 4.
            assert gpu.metadata_stats() == (33, 3288 * 2)
    finally:
        gpu.close()


def test_full_size_matrix_loads_and_matches_oracle(tmp_path):
    """BASELINE config 1's down projection (5120x17408 Q4/g64, BF16 metadata)
    written as an MLX checkpoint, loaded into a "bf16" device and multiplied:
    the GEMV on the loaded buffers meets the gate."""
    rows, cols = synth.MLP_SHAPES["down"]
    m = synth.q4_bf16_matrix(rows, cols, synth.DEFAULT_SEED, tag="down")
    name = "model.layers.0.mlp.down_proj"
    write_config(tmp_path, quantization={"bits": 4, "group_size": 64})
    write_tensor_file(tmp_path / "model.safetensors", [
        (f"{name}.weight", "U32", [rows, cols // 8], m.w.tobytes()),
        (f"{name}.scales", "BF16", [rows, cols // 64], m.s.tobytes()),
        (f"{name}.biases", "BF16", [rows, cols // 64], m.b.tobytes()),
    ])
    gpu = qmr.Gpu("aligned", metadata="bf16")
    try:
        with qmr.Checkpoint(tmp_path) as cp:
            t = time.perf_counter()
            dm = cp.load(gpu, name, rows, cols)
            print(f"loaded {name} [{rows},{cols}] in {1e3 * (time.perf_counter() - t):.1f} ms", flush=True)
            assert dm.metadata_bf16
            assert np.array_equal(dm.scales.read(np.uint16, m.s.size), m.s)
            x = synth.activations(cols, 1, synth.DEFAULT_SEED, tag="ck")
            want = oracle.matmul_f64(m.w, m.s, m.b, "bf16", x, rows, cols, 4, 64, 1, 8)
            assert_gate(_product(gpu, dm, x, 1), want, "loaded down projection")
    finally:
        gpu.close()


def test_dense_matrix_loads_as_f16(tmp_path):
    """A dense F32 matrix is uploaded as F16 (Matrix::load, dense case) and
    multiplies through matvec_f16 like the reference's known answer
    (src/gpu.rs:1699-1708)."""
    write_config(tmp_path)
    vals = np.array([1, 2, 3, 4, -1, 0, 1, 2], np.float32)
    write_tensor_file(tmp_path / "model.safetensors", [("model.w.weight", "F32", [2, 4], vals.tobytes())])
    gpu = qmr.Gpu("aligned")
    try:
        with qmr.Checkpoint(tmp_path) as cp:
            m = cp.load(gpu, "model.w", 2, 4)
            assert (m.bits, m.group, m.scales, m.biases) == (16, 0, None, None)
            assert m.weight.read(np.uint16, 8).tolist() == vals.astype(np.float16).view(np.uint16).tolist()
            x = gpu.upload_f32([1, 2, 3, 4])
            y = gpu.alloc_f32(2)
            gpu.dispatch("matvec_f16", [m.weight, x, y], [2, 4])
            np.testing.assert_allclose(gpu.read_f32(y, 2), [30, 10], rtol=3e-5)
    finally:
        gpu.close()


def test_load_rejects_wrong_shape_without_allocating(tmp_path):
    names = _fixture_checkpoint(tmp_path, "q4bf16")
    name, rows, cols = names[0]
    gpu = qmr.Gpu("aligned", metadata="bf16")
    try:
        with qmr.Checkpoint(tmp_path) as cp:
            with pytest.raises(qmr.QmrError, match=rf"expected \[{rows + 1},{cols}\], got \[{rows},{cols}\]"):
                cp.load(gpu, name, rows + 1, cols)
            with pytest.raises(qmr.QmrError, match="loading model.nothing: missing tensor model.nothing.weight"):
                cp.load(gpu, "model.nothing", 1, 1)
            assert gpu.metadata_stats()[0] == 0
    finally:
        gpu.close()


@pytest.mark.parametrize("mode", ["bf16", "f32"])
@pytest.mark.parametrize("bad", [0x7F80, 0xFF80, 0x7FC1, 0xFFFF])
def test_non_finite_bf16_metadata_is_rejected(tmp_path, mode, bad):
    """Inf and NaN BF16 scales or biases fail the load on both metadata paths
    (Checkpoint::quant_values, src/weights.rs:416-425), including the device
    that would keep the stored BF16 bits."""
    write_config(tmp_path, quantization={"bits": 4, "group_size": 32})
    good = np.full(2, 0x3C00, np.uint16)
    for which in ("scales", "biases"):
        s, b = good.copy(), good.copy()
        (s if which == "scales" else b)[1] = bad
        write_tensor_file(tmp_path / "model.safetensors", [
            ("model.w.weight", "U32", [2, 4], np.arange(8, dtype=np.uint32).tobytes()),
            ("model.w.scales", "BF16", [2, 1], s.tobytes()),
            ("model.w.biases", "BF16", [2, 1], b.tobytes()),
        ])
        gpu = qmr.Gpu("aligned", metadata=mode)
        try:
            with qmr.Checkpoint(tmp_path) as cp:
                with pytest.raises(qmr.QmrError, match=f"model.w.{which} contains non-finite values"):
                    cp.load(gpu, "model.w", 2, 32)
            assert gpu.metadata_stats()[0] == 0
        finally:
            gpu.close()

"""Shared input builders and checks for the GPU parity tests."""
from __future__ import annotations

import json
import struct

import numpy as np

import oracle
import qmr

# BASELINE gate: rel-L2 <= 1e-5 and max-abs <= 1e-4 * max|y64|.
GATE_REL_L2 = 1e-5
GATE_REL_MAX = 1e-4


def xorshift_words(seed: int, n: int) -> np.ndarray:
    """The reference's xorshift32 word stream (tests/quantized.rs:18-30)."""
    out = np.empty(n, np.uint32)
    s = seed & 0xFFFFFFFF
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = s
    return out


def rotl(v: int, r: int) -> int:
    v &= 0xFFFFFFFF
    return ((v << r) | (v >> (32 - r))) & 0xFFFFFFFF


def reference_metadata(n: int) -> tuple[np.ndarray, np.ndarray]:
    """tests/quantized.rs:31-36: scale 0.001*(1 + i%11), bias -0.07 + (i%9)*0.003."""
    i = np.arange(n)
    s = (0.001 * (1 + i % 11)).astype(np.float32)
    b = (-0.07 + (i % 9).astype(np.float32) * np.float32(0.003)).astype(np.float32)
    return s, b


def reference_x(n: int) -> np.ndarray:
    """tests/quantized.rs:37-39: ((i*13 % 101) - 50) / 50."""
    i = np.arange(n)
    return (((i * 13) % 101).astype(np.float32) - 50.0) / 50.0


def to_bf16_truncated(v: np.ndarray) -> np.ndarray:
    """tests/bf16_metadata.rs:24-36: FP32 bits with the low half cleared."""
    return ((np.asarray(v, np.float32).view(np.uint32) >> 16)).astype(np.uint16)


def assert_close_ref(got, want, atol, rtol, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bad = np.abs(got - want) >= atol + rtol * np.abs(want)
    if bad.any():
        i = int(np.argmax(bad))
        raise AssertionError(f"{what}: index {i}: {got[i]} vs {want[i]} ({bad.sum()} bad)")


def assert_gate(y_gpu, y64, what=""):
    rel_l2, rel_max = oracle.gate(y_gpu, y64)
    assert rel_l2 <= GATE_REL_L2 and rel_max <= GATE_REL_MAX, \
        f"{what}: rel_l2={rel_l2:.3e} rel_max={rel_max:.3e}"
    return rel_l2, rel_max


def upload_matrix(gpu: qmr.Gpu, w, s, b):
    return gpu.upload_bytes(np.ascontiguousarray(w)), gpu.upload_bytes(np.ascontiguousarray(s)), \
        gpu.upload_bytes(np.ascontiguousarray(b))


def run_affine(gpu: qmr.Gpu, name: str, w, s, b, x, rows, cols, bits, group, batch=1):
    """One matvec/matmul dispatch; returns y as FP32 [batch*rows]."""
    wb, sb, bb = upload_matrix(gpu, w, s, b)
    xb = gpu.upload_f32(np.ascontiguousarray(x, np.float32).ravel())
    yb = gpu.alloc_f32(batch * rows)
    params = [rows, cols, bits, group] + ([batch] if name.startswith("matmul") else [])
    gpu.dispatch(name, [wb, sb, bb, xb, yb], params)
    return gpu.read_f32(yb, batch * rows)


# ---- safetensors checkpoints written by the tests

def write_tensor_file(path: Path, tensors, metadata=None) -> None:
    """Safetensors writer in the shape of the reference's test helper
    (src/weights.rs:759-776): tensors laid out in order, offsets relative to
    the data section."""
    header, data = {}, b""
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, dtype, shape, payload in tensors:
        start = len(data)
        data += payload
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [start, len(data)]}
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + data)


def write_raw(path: Path, header: bytes, data: bytes = b"") -> None:
    path.write_bytes(struct.pack("<Q", len(header)) + header + data)


def write_config(d: Path, **extra) -> None:
    cfg = {"model_type": "qwen3_5_text", "hidden_size": 8}
    cfg.update(extra)
    (d / "config.json").write_text(json.dumps(cfg))

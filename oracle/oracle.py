"""ctypes wrapper of liboracle.so (qmr_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product library never uses
it. Builds the library with `make -C oracle` when it is missing.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
META_KIND = {"f32": 0, "bf16": 1, "f16": 2}

_lib: Optional[C.CDLL] = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            subprocess.run(["make", "-C", str(HERE), "liboracle.so"], check=True,
                           capture_output=True)
        L = C.CDLL(str(LIB))
        vp, sz = C.c_void_p, C.c_size_t
        L.oracle_bf16_to_f32.restype = C.c_float
        L.oracle_bf16_to_f32.argtypes = [C.c_uint16]
        L.oracle_f16_to_f32.restype = C.c_float
        L.oracle_f16_to_f32.argtypes = [C.c_uint16]
        L.oracle_code.restype = C.c_uint32
        L.oracle_code.argtypes = [vp, sz, C.c_uint32, sz, sz]
        L.oracle_dequant_row.restype = None
        L.oracle_dequant_row.argtypes = [vp, vp, vp, C.c_int, sz, sz, C.c_uint32, sz, vp]
        for name in ("oracle_matmul_f64", "oracle_matmul_f32"):
            fn = getattr(L, name)
            fn.restype = C.c_int
            fn.argtypes = [vp, vp, vp, C.c_int, vp, vp, sz, sz, C.c_uint32, sz, sz, C.c_int]
        L.oracle_pack_bf16_exact.restype = C.c_int
        L.oracle_pack_bf16_exact.argtypes = [vp, sz, vp]
        L.oracle_dense_f16_f64.restype = C.c_int
        L.oracle_dense_f16_f64.argtypes = [vp, vp, vp, sz, sz, sz]
        _lib = L
    return _lib


def _meta_array(v: np.ndarray, kind: str) -> np.ndarray:
    return np.ascontiguousarray(v, dtype=np.float32 if kind == "f32" else np.uint16)


def _check_sizes(w, x, rows, cols, bits, group, batch) -> None:
    """Host-side size check for valid shapes; invalid shapes are left to the
    C oracle's own validation, which rejects them."""
    if bits in (4, 8) and group > 0 and rows > 0 and cols > 0 and cols % (32 // bits) == 0:
        if x.size < batch * cols or w.size < rows * cols * bits // 32:
            raise ValueError("oracle: arrays smaller than the shape")


def matmul_f64(w, s, b, kind: str, x, rows: int, cols: int, bits: int, group: int,
               batch: int = 1, threads: int = 1) -> np.ndarray:
    """FP64 oracle: y[t*rows + r] (tests/quantized.rs:39-51, tests/batch_matrix.rs:35-49)."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s, b = _meta_array(s, kind), _meta_array(b, kind)
    x = np.ascontiguousarray(x, dtype=np.float32)
    _check_sizes(w, x, rows, cols, bits, group, batch)
    y = np.empty(batch * rows, dtype=np.float64)
    rc = lib().oracle_matmul_f64(w.ctypes.data, s.ctypes.data, b.ctypes.data, META_KIND[kind],
                                 x.ctypes.data, y.ctypes.data, rows, cols, bits, group, batch,
                                 threads)
    if rc != 0:
        raise ValueError("oracle: invalid shape")
    return y


def matmul_f32(w, s, b, kind: str, x, rows: int, cols: int, bits: int, group: int,
               batch: int = 1, threads: int = 1) -> np.ndarray:
    """FP32-accumulating CPU baseline (same per-weight dequantise-then-multiply)."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s, b = _meta_array(s, kind), _meta_array(b, kind)
    x = np.ascontiguousarray(x, dtype=np.float32)
    _check_sizes(w, x, rows, cols, bits, group, batch)
    y = np.empty(batch * rows, dtype=np.float32)
    rc = lib().oracle_matmul_f32(w.ctypes.data, s.ctypes.data, b.ctypes.data, META_KIND[kind],
                                 x.ctypes.data, y.ctypes.data, rows, cols, bits, group, batch,
                                 threads)
    if rc != 0:
        raise ValueError("oracle: invalid shape")
    return y


def dequant_row(w, s, b, kind: str, row: int, cols: int, bits: int, group: int) -> np.ndarray:
    """RN32(q*s + b) for one row (the embedding kernels)."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s, b = _meta_array(s, kind), _meta_array(b, kind)
    out = np.empty(cols, dtype=np.float32)
    lib().oracle_dequant_row(w.ctypes.data, s.ctypes.data, b.ctypes.data, META_KIND[kind], row,
                             cols, bits, group, out.ctypes.data)
    return out


def code(w, cols: int, bits: int, row: int, col: int) -> int:
    w = np.ascontiguousarray(w, dtype=np.uint32)
    return int(lib().oracle_code(w.ctypes.data, cols, bits, row, col))


def f16_to_f32(h: int) -> float:
    return float(lib().oracle_f16_to_f32(h))


def bf16_to_f32(h: int) -> float:
    return float(lib().oracle_bf16_to_f32(h))


def pack_bf16_exact(values) -> Optional[np.ndarray]:
    v = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(v.size, dtype=np.uint16)
    return out if lib().oracle_pack_bf16_exact(v.ctypes.data, v.size, out.ctypes.data) else None


def dense_f16_f64(w16, x, rows: int, cols: int, batch: int = 1) -> np.ndarray:
    w16 = np.ascontiguousarray(w16, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(batch * rows, dtype=np.float64)
    if lib().oracle_dense_f16_f64(w16.ctypes.data, x.ctypes.data, y.ctypes.data, rows, cols,
                                  batch) != 0:
        raise ValueError("oracle: invalid shape")
    return y


# ---- the decoder layer's elementwise steps around the products (FP64) ----


def rms_norm_f64(x, w, eps: float) -> np.ndarray:
    """kernels/qwen.metal:78-86 (rms_norm) per row of x [batch][n]:
    y = x * w / sqrt(mean(x^2) + eps)."""
    x = np.asarray(x, np.float64)
    x2 = x.reshape(-1, x.shape[-1])
    inv = 1.0 / np.sqrt(np.mean(x2 * x2, axis=1, keepdims=True) + float(eps))
    return (x2 * inv * np.asarray(w, np.float64)).reshape(x.shape)


def swiglu_f64(g, u) -> np.ndarray:
    """kernels/qwen.metal:32-33,91-94 (swiglu): silu(g) * u, silu(g) = g / (1 + e^-g)."""
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)


def mlp_gate_up_f64(gate_m, up_m, kind: str, x, norm_w, eps: float, rows: int, cols: int, bits: int,
                    group: int, batch: int = 1, threads: int = 1) -> np.ndarray:
    """The decoder MLP's first half (src/engine.rs:748-764): rms_norm, the
    gate and up products of the normalised x, then swiglu. gate_m and up_m
    are (w, s, b) triples; the products are the FP64 oracle of matmul_f64
    applied to the FP64 normalised x rounded to FP32, the precision the
    reference hands its GEMV."""
    n = rms_norm_f64(np.asarray(x, np.float32).reshape(batch, cols), norm_w, eps).astype(np.float32)
    g = matmul_f64(*gate_m, kind, n, rows, cols, bits, group, batch, threads)
    u = matmul_f64(*up_m, kind, n, rows, cols, bits, group, batch, threads)
    return swiglu_f64(g, u)


def matmul_add_f64(w, s, b, kind: str, x, r, rows: int, cols: int, bits: int, group: int,
                   batch: int = 1, threads: int = 1) -> np.ndarray:
    """A product followed by the reference's add (kernels/qwen.metal:87-90,
    src/engine.rs:765): y = r + W x."""
    return np.asarray(r, np.float64).ravel() + matmul_f64(w, s, b, kind, x, rows, cols, bits, group, batch,
                                                          threads)


def gate(y_gpu: np.ndarray, y64: np.ndarray) -> tuple[float, float]:
    """(relative L2, max-abs / max|y64|) of a GPU result against the FP64 oracle."""
    y = np.asarray(y_gpu, dtype=np.float64)
    d = y - y64
    rel_l2 = float(np.linalg.norm(d) / max(np.linalg.norm(y64), 1e-300))
    rel_max = float(np.max(np.abs(d)) / max(np.max(np.abs(y64)), 1e-300))
    return rel_l2, rel_max

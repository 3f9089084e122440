"""Seeded synthetic inputs for the packed-affine benchmark configurations.

Distributions (one generator per tensor, numpy PCG64 seeded by
(seed, tensor tag), so every tensor is reproducible on its own):
  Q4/g64, BF16 metadata: codes uniform 0..15 (8 per little-endian u32),
      scale = BF16(U(0.002, 0.02)), bias = BF16(-8*scale + N(0, 1e-3)).
  Q8/g64, F16 metadata:  codes uniform 0..255 (4 per u32),
      scale = F16(U(1e-4, 2e-3)), bias = F16(-128*scale) (exact in F16).
  Activations: FP32 N(0, 1), token-major [batch][cols].
Rounding to BF16 and F16 is round-to-nearest-even.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass
from typing import Optional

import numpy as np


def _rng(seed: int, tag: str) -> np.random.Generator:
    h = int.from_bytes(hashlib.sha256(tag.encode()).digest()[:8], "little")
    return np.random.default_rng([seed & 0xFFFFFFFFFFFFFFFF, h])


def f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """Round FP32 to BF16 (nearest, ties to even); returns u16 bit patterns."""
    bits = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint32) << 16).view(np.float32)


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


@dataclass
class PackedMatrix:
    rows: int
    cols: int
    bits: int
    group: int
    meta: str            # "bf16" | "f16" | "f32"
    w: np.ndarray        # u32 [rows * cols*bits/32]
    s: np.ndarray        # u16 bit patterns (bf16/f16) or f32, [rows * cols/group]
    b: np.ndarray

    @property
    def nbytes(self) -> int:
        return self.w.nbytes + self.s.nbytes + self.b.nbytes

    def scales_f32(self) -> np.ndarray:
        return _meta_f32(self.s, self.meta)

    def biases_f32(self) -> np.ndarray:
        return _meta_f32(self.b, self.meta)


def _meta_f32(v: np.ndarray, kind: str) -> np.ndarray:
    if kind == "bf16":
        return bf16_bits_to_f32(v)
    if kind == "f16":
        return f16_bits_to_f32(v)
    return np.asarray(v, dtype=np.float32)


def q4_bf16_matrix(rows: int, cols: int, seed: int, tag: str = "q4") -> PackedMatrix:
    """Q4/g64 with BF16 metadata (configs 0-2, 4 and the vocabulary head)."""
    group = 64
    words = rows * cols // 8
    w = _rng(seed, f"{tag}:codes").integers(0, 2**32, size=words, dtype=np.uint32)
    n = rows * cols // group
    r = _rng(seed, f"{tag}:meta")
    scale = f32_to_bf16_bits(r.uniform(0.002, 0.02, size=n).astype(np.float32))
    sf = bf16_bits_to_f32(scale)
    bias = f32_to_bf16_bits((-8.0 * sf.astype(np.float64) + r.normal(0.0, 1e-3, size=n)).astype(np.float32))
    return PackedMatrix(rows, cols, 4, group, "bf16", w, scale, bias)


def q8_f16_matrix(rows: int, cols: int, seed: int, tag: str = "q8") -> PackedMatrix:
    """Q8/g64 with F16 metadata (config 3)."""
    group = 64
    words = rows * cols // 4
    w = _rng(seed, f"{tag}:codes").integers(0, 2**32, size=words, dtype=np.uint32)
    n = rows * cols // group
    r = _rng(seed, f"{tag}:meta")
    scale = r.uniform(1e-4, 2e-3, size=n).astype(np.float16)
    bias = (-128.0 * scale.astype(np.float32)).astype(np.float16)
    assert np.array_equal(bias.astype(np.float32), -128.0 * scale.astype(np.float32))
    return PackedMatrix(rows, cols, 8, group, "f16", w, scale.view(np.uint16), bias.view(np.uint16))


def to_f32_metadata(m: PackedMatrix) -> PackedMatrix:
    """The same matrix with metadata expanded to FP32 (the reference's storage)."""
    return PackedMatrix(m.rows, m.cols, m.bits, m.group, "f32", m.w,
                        m.scales_f32().copy(), m.biases_f32().copy())


def activations(cols: int, batch: int, seed: int, tag: str = "x") -> np.ndarray:
    """FP32 N(0,1) activations, token-major [batch][cols]."""
    return _rng(seed, f"{tag}:{cols}x{batch}").standard_normal((batch, cols)).astype(np.float32)


# The BASELINE configurations (rows x cols = N_out x K).
MLP_SHAPES = {"gate_up": (17408, 5120), "down": (5120, 17408)}
HEAD_SHAPE = (151936, 5120)
Q8_SHAPE = (5120, 5120)
CONFIG0_SHAPE = (1024, 1024)
DEFAULT_SEED = 20261201


def algorithmic_bytes(m: PackedMatrix, batch: int) -> int:
    """codes + scales + biases + x + y (the roofline's byte count)."""
    return m.nbytes + 4 * batch * m.cols + 4 * batch * m.rows


def describe(m: PackedMatrix, batch: Optional[int] = None) -> str:
    meta = {"bf16": "BF16", "f16": "F16", "f32": "FP32"}[m.meta]
    s = f"Q{m.bits}/g{m.group} {meta}-meta {m.rows}x{m.cols}"
    return s if batch is None else f"{s} B={batch}"

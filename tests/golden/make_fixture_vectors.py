"""Extracts the reference's MLX-format test fixtures into tests/golden/.

Reads, as data only, three safetensors files the reference's own tests hold:
  tests/fixtures/tiny/model.safetensors       dense F16 matrices (originals)
  tests/fixtures/tiny-q4/model.safetensors    Q4/g32, F16 scales/biases, U32 codes
  tests/fixtures/tiny-bf16/model.safetensors  Q4/g32, BF16 scales/biases, U32 codes
and writes tests/golden/mlx_fixtures.npz with, per 2-D matrix, the original
F16 bits, the packed words and the raw 16-bit metadata of both quantised
checkpoints. The files are parsed directly (8-byte little-endian header
length, JSON header, raw little-endian payload); nothing is executed.

Run once in a container where the reference is mounted:
    python tests/golden/make_fixture_vectors.py /root/reference
"""
from __future__ import annotations

import json
import struct
import sys
from pathlib import Path

import numpy as np

DTYPES = {"F16": np.uint16, "BF16": np.uint16, "U32": np.uint32, "F32": np.float32}


def read_safetensors(path: Path) -> dict[str, tuple[str, list[int], np.ndarray]]:
    data = path.read_bytes()
    (n,) = struct.unpack("<Q", data[:8])
    header = json.loads(data[8:8 + n])
    body = data[8 + n:]
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        start, end = meta["data_offsets"]
        arr = np.frombuffer(body[start:end], dtype=DTYPES[meta["dtype"]]).copy()
        out[name] = (meta["dtype"], meta["shape"], arr)
    return out


def main(reference: Path) -> None:
    fx = reference / "tests" / "fixtures"
    dense = read_safetensors(fx / "tiny" / "model.safetensors")
    q4 = read_safetensors(fx / "tiny-q4" / "model.safetensors")
    bf = read_safetensors(fx / "tiny-bf16" / "model.safetensors")
    arrays: dict[str, np.ndarray] = {}
    names = []
    for name, (dtype, shape, arr) in sorted(dense.items()):
        if len(shape) != 2 or not name.endswith(".weight") or dtype != "F16":
            continue
        module = "language_model." + name[: -len(".weight")]
        if module + ".weight" not in q4:
            continue
        rows, cols = shape
        key = name[: -len(".weight")].replace(".", "/")
        arrays[f"{key}/shape"] = np.array([rows, cols], dtype=np.int64)
        arrays[f"{key}/f16"] = arr
        for tag, ck in (("q4f16", q4), ("q4bf16", bf)):
            wd, wshape, w = ck[module + ".weight"]
            sd, _, s = ck[module + ".scales"]
            bd, _, b = ck[module + ".biases"]
            assert wd == "U32" and wshape == [rows, cols // 8]
            arrays[f"{key}/{tag}/w"] = w
            arrays[f"{key}/{tag}/s"] = s
            arrays[f"{key}/{tag}/b"] = b
            arrays[f"{key}/{tag}/meta"] = np.frombuffer(sd.encode(), dtype=np.uint8)
            assert sd == bd
        names.append(key)
    out = Path(__file__).resolve().parent / "mlx_fixtures.npz"
    np.savez_compressed(out, **arrays)
    print(f"wrote {len(names)} matrices to {out}")


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))

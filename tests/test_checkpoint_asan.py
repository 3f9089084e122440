"""The checkpoint loader's host code under AddressSanitizer and
UndefinedBehaviorSanitizer (g++, CPU only): a driver built from
csrc/checkpoint.cpp and csrc/contract.cpp, with the device-facing entry
points stubbed, opens valid checkpoints (the MLX fixture matrices) and
hundreds of corrupted ones and reads every matrix; any sanitizer report
fails the test."""
from __future__ import annotations

import json
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

from helpers import write_config, write_tensor_file

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "qwen-mlx-runner_amd" / "csrc"


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ is not available")
    out = tmp_path_factory.mktemp("asan") / "checkpoint_driver"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", str(ROOT / "tests" / "asan" / "checkpoint_driver.cpp"),
           str(CSRC / "checkpoint.cpp"), str(CSRC / "contract.cpp"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    return out


def _corpus(root: Path) -> list[str]:
    z = np.load(Path(__file__).resolve().parent / "golden" / "mlx_fixtures.npz")
    keys = sorted({k.rsplit("/", 1)[0] for k in z.files if k.endswith("/shape")})[:6]
    tensors = []
    for key in keys:
        rows, cols = (int(v) for v in z[f"{key}/shape"])
        raw = "language_model." + key.replace("/", ".")
        tensors += [(raw + ".weight", "U32", [rows, cols // 8], z[f"{key}/q4bf16/w"].tobytes()),
                    (raw + ".scales", "BF16", [rows, cols // 32], z[f"{key}/q4bf16/s"].tobytes()),
                    (raw + ".biases", "BF16", [rows, cols // 32], z[f"{key}/q4bf16/b"].tobytes()),
                    (key.replace("/", ".") + "_dense.weight", "F16", [rows, cols], z[f"{key}/f16"].tobytes())]
    dirs = []
    good = root / "good"
    good.mkdir()
    write_config(good, quantization={"bits": 4, "group_size": 32})
    write_tensor_file(good / "model.safetensors", tensors)
    dirs.append(str(good))
    blob = (good / "model.safetensors").read_bytes()
    (n,) = struct.unpack("<Q", blob[:8])
    rng = np.random.default_rng(0)
    for i in range(300):
        d = root / f"bad{i}"
        d.mkdir()
        write_config(d, quantization={"bits": int(rng.choice([4, 8])), "group_size": int(rng.choice([8, 32, 64]))})
        b = bytearray(blob)
        kind = i % 4
        if kind == 0:    # flip header bytes
            for _ in range(int(rng.integers(1, 6))):
                b[8 + int(rng.integers(0, n))] = int(rng.integers(32, 127))
        elif kind == 1:  # truncate anywhere
            b = b[: int(rng.integers(0, len(b)))]
        elif kind == 2:  # a wrong header length
            b[:8] = struct.pack("<Q", int(rng.integers(0, 2 * n)))
        else:            # corrupt data bytes (non-finite metadata, odd codes)
            for _ in range(int(rng.integers(1, 50))):
                b[8 + n + int(rng.integers(0, len(b) - 8 - n))] = int(rng.integers(0, 256))
        (d / "model.safetensors").write_bytes(bytes(b))
        dirs.append(str(d))
    names = [k.replace("/", ".") for k in keys] + [k.replace("/", ".") + "_dense" for k in keys] + ["lm_head"]
    return dirs + ["--"] + names


def test_loader_host_code_is_clean_under_sanitizers(driver, tmp_path):
    args = _corpus(tmp_path)
    res = subprocess.run([str(driver), *args], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0 and "ERROR: AddressSanitizer" not in res.stderr and "runtime error" not in res.stderr, \
        res.stderr[-3000:]
    opened, read = (int(v) for v in res.stdout.split()[1::2])
    assert opened >= 1 and read >= 12, res.stdout

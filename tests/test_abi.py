"""The C ABI library loads on a CPU-only host and exports exactly what
include/*.h declare; the generator reproduces the documented
distributions. No GPU compute happens here."""
import ctypes
import os
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import qmr
import qmr.synth as synth

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"\b(qmr_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    assert [h.name for h in HEADERS] == ["qmr.h", "qmr_checkpoint.h"]
    names = declared_functions()
    assert len(names) >= 45
    L = ctypes.CDLL(str(qmr.LIB_PATH))
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # The binding covers the same set.
    assert sorted(qmr.EXPORTED_SYMBOLS) == names


def test_exported_dynamic_symbols_are_c_linkage():
    out = subprocess.run(["nm", "-D", "--defined-only", str(qmr.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for n in declared_functions():
        assert n in exported, n


def test_device_open_without_gpu_fails_loudly():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present; covered by the gpu tests")
    with pytest.raises(qmr.QmrError) as e:
        qmr.Gpu()
    assert e.value.code == qmr.QMR_ERR_DEVICE
    assert "gfx950" in str(e.value)


def test_invalid_device_options_are_rejected_before_device_access():
    for kw in ({"variant": "fast"}, {"metadata": "f16"}, {"block_matmul": "LEGACY"},
               {"block_delta": "auto"}):
        with pytest.raises(qmr.QmrError):
            qmr.Gpu(**kw)


def test_q4_generator_distributions():
    m = synth.q4_bf16_matrix(256, 4096, 1, tag="t")
    codes = np.stack([(m.w >> (4 * i)) & 15 for i in range(8)])
    counts = np.bincount(codes.ravel(), minlength=16)
    assert counts.min() > 0.9 * counts.mean()
    s, b = m.scales_f32(), m.biases_f32()
    assert s.min() >= 0.0019 and s.max() <= 0.0201
    assert np.abs(b + 8 * s).max() < 6e-3  # N(0, 1e-3) plus BF16 rounding
    assert (m.s.astype(np.uint32) << 16).view(np.float32).tolist() == s.tolist()
    again = synth.q4_bf16_matrix(256, 4096, 1, tag="t")
    assert np.array_equal(again.w, m.w) and np.array_equal(again.s, m.s)


def test_q8_generator_bias_is_exact_f16():
    m = synth.q8_f16_matrix(64, 1024, 2)
    s, b = m.scales_f32(), m.biases_f32()
    assert np.array_equal(b, -128.0 * s)
    assert s.min() >= 9.9e-5 and s.max() <= 2.001e-3


def test_bf16_rounding_is_nearest_even():
    v = np.array([1.0, 1.00390625, 1.0078125 + 2**-9, 1.01171875, -3.0], np.float32)
    got = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(v))
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 2^-7 + 2^-9 is below the midpoint
    # -> 1 + 2^-7; 1 + 3*2^-8 is a tie -> even (1 + 2^-6).
    assert got.tolist() == [1.0, 1.0, 1.0078125, 1.015625, -3.0]

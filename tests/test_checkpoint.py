"""The MLX checkpoint loader (include/qmr_checkpoint.h) on the CPU.

Restates the reference's own loader tests (src/weights.rs:816-1115), loads the
genuine MLX bytes of its tiny-q4 / tiny-bf16 fixtures (extracted, as data, to
tests/golden/mlx_fixtures.npz) back through safetensors files written here,
and pins the F16 conversion of dense matrices against numpy's IEEE
round-to-nearest-even. None of these calls touches a GPU.
"""
from __future__ import annotations

import json
import os
import struct
from pathlib import Path

import numpy as np
import pytest

import qmr
from helpers import write_config, write_raw, write_tensor_file

GOLDEN = Path(__file__).resolve().parent / "golden"


def u32(*v) -> bytes:
    return struct.pack(f"<{len(v)}I", *v)


def u16(*v) -> bytes:
    return struct.pack(f"<{len(v)}H", *v)


def f32(*v) -> bytes:
    return struct.pack(f"<{len(v)}f", *v)


def rejected(d: Path, needle: str = "") -> str:
    with pytest.raises(qmr.QmrError) as e:
        qmr.Checkpoint(d)
    assert needle in str(e.value), str(e.value)
    return str(e.value)


# ----------------------------------------------- the reference's loader tests


def test_packed_nibbles_keep_low_to_high_order_and_per_layer_quant(tmp_path):
    """src/weights.rs:816-871: an 8-bit default with a 4-bit/g8 override for
    one module; the word 0x76543210 decodes low nibble first."""
    write_config(tmp_path, quantization={
        "bits": 8, "group_size": 8, "mode": "affine",
        "language_model.model.layers.0.mlp.gate_proj": {"bits": 4, "group_size": 8}})
    p = "language_model.model.layers.0.mlp.gate_proj"
    write_tensor_file(tmp_path / "model.safetensors", [
        (f"{p}.weight", "U32", [1, 1], u32(0x76543210)),
        (f"{p}.scales", "F16", [1, 1], u16(0x3800)),
        (f"{p}.biases", "F16", [1, 1], u16(0xBC00)),
    ])
    with qmr.Checkpoint(tmp_path) as cp:
        m = cp.matrix("model.layers.0.mlp.gate_proj")
        assert isinstance(m, qmr.PackedData)
        assert (m.cols, m.bits, m.group_size) == (8, 4, 8)
        assert m.weights[0] == 0x76543210
        assert m.scales.tolist() == [0.5] and m.biases.tolist() == [-1.0]
        decoded = [((int(m.weights[0]) >> (4 * i)) & 15) * m.scales[0] + m.biases[0] for i in range(8)]
        assert decoded == [-1.0, -0.5, 0.0, 0.5, 1.0, 1.5, 2.0, 2.5]
        # The same matrix under its ".weight" name and under the raw prefix.
        assert cp.matrix_info(f"{p}.weight") == cp.matrix_info("model.layers.0.mlp.gate_proj")


def test_truncated_tensor_and_index_traversal_are_rejected(tmp_path):
    """src/weights.rs:873-893."""
    write_config(tmp_path)
    write_tensor_file(tmp_path / "model.safetensors", [("model.norm.weight", "F32", [2], f32(1.0))])
    rejected(tmp_path, "byte length mismatch")
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {"model.norm.weight": "../other.safetensors"}}))
    rejected(tmp_path, "unsafe shard filename")


def test_indexed_shards_must_match_named_file(tmp_path):
    """src/weights.rs:1021-1048, with a dense matrix where the reference reads
    a norm vector (vectors are model-level and not on this path)."""
    write_config(tmp_path)
    write_tensor_file(tmp_path / "a.safetensors", [("model.layers.0.mlp.up_proj.weight", "F32", [1, 1],
                                                    f32(1.0))])
    index = tmp_path / "model.safetensors.index.json"
    index.write_text(json.dumps({"weight_map": {"model.layers.0.mlp.up_proj.weight": "a.safetensors"}}))
    with qmr.Checkpoint(tmp_path) as cp:
        d = cp.matrix("model.layers.0.mlp.up_proj")
        assert isinstance(d, qmr.DenseData) and d.values.tolist() == [0x3C00]
    index.write_text(json.dumps({"weight_map": {"model.layers.0.mlp.up_proj.weight": "b.safetensors"}}))
    rejected(tmp_path)


def test_safetensors_rejects_unindexed_data_bytes(tmp_path):
    """src/weights.rs:1074-1091."""
    write_config(tmp_path)
    path = tmp_path / "model.safetensors"
    write_tensor_file(path, [("model.norm.weight", "F32", [1], f32(0.0))])
    path.write_bytes(path.read_bytes() + b"\0")
    rejected(tmp_path, "unindexed trailing bytes")


def test_safetensors_rejects_non_string_metadata(tmp_path):
    """src/weights.rs:1093-1102."""
    write_config(tmp_path)
    write_raw(tmp_path / "model.safetensors", json.dumps({"__metadata__": {"producer": 42}}).encode())
    rejected(tmp_path, "invalid safetensors metadata value")


def test_safetensors_rejects_duplicate_json_keys(tmp_path):
    """src/weights.rs:1104-1114: a duplicate key inside a tensor entry."""
    write_config(tmp_path)
    header = (b'{"model.norm.weight":{"dtype":"F32","shape":[1],"data_offsets":[0,4],'
              b'"shape":[1]}}')
    write_raw(tmp_path / "model.safetensors", header, f32(0.0))
    rejected(tmp_path, "duplicate key")


# ------------------------------------------------ genuine MLX fixture bytes


def _fixture():
    return np.load(GOLDEN / "mlx_fixtures.npz")


def _matrix_names(z):
    return sorted({k.rsplit("/", 1)[0] for k in z.files if k.endswith("/shape")})


def _raw_name(key: str) -> str:
    """The fixtures' tensor names are language_model.<canonical name>."""
    return "language_model." + key.replace("/", ".")


def _expand(bits: np.ndarray, kind: str) -> np.ndarray:
    if kind == "F16":
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("tag", ["q4f16", "q4bf16"])
def test_mlx_fixture_checkpoints_load_words_and_exact_metadata(tmp_path, tag):
    """The tiny-q4 (F16 metadata) and tiny-bf16 (BF16 metadata) fixtures'
    33 packed matrices: words unchanged, metadata expanded exactly, and the
    dequantised weights within the quantiser's rounding bound of the
    original F16 matrices (tests/fixtures/tiny)."""
    z = _fixture()
    names = _matrix_names(z)
    tensors = []
    for key in names:
        rows, cols = (int(v) for v in z[f"{key}/shape"])
        kind = z[f"{key}/{tag}/meta"].tobytes().decode()
        tensors += [(_raw_name(key) + ".weight", "U32", [rows, cols // 8], z[f"{key}/{tag}/w"].tobytes()),
                    (_raw_name(key) + ".scales", kind, [rows, cols // 32], z[f"{key}/{tag}/s"].tobytes()),
                    (_raw_name(key) + ".biases", kind, [rows, cols // 32], z[f"{key}/{tag}/b"].tobytes())]
    write_config(tmp_path, quantization={"bits": 4, "group_size": 32, "mode": "affine"})
    write_tensor_file(tmp_path / "model.safetensors", tensors)
    with qmr.Checkpoint(tmp_path) as cp:
        assert len(cp) == 3 * len(names) == 99
        for key in names:
            rows, cols = (int(v) for v in z[f"{key}/shape"])
            kind = z[f"{key}/{tag}/meta"].tobytes().decode()
            name = key.replace("/", ".")
            info = cp.matrix_info(name)
            assert info == qmr.MatrixInfo(True, rows, cols, 4, 32, "U32", kind), key
            m = cp.matrix(name)
            assert np.array_equal(m.weights, z[f"{key}/{tag}/w"]), key
            s, b = _expand(z[f"{key}/{tag}/s"], kind), _expand(z[f"{key}/{tag}/b"], kind)
            assert np.array_equal(m.scales.view(np.uint32), s.view(np.uint32)), key
            assert np.array_equal(m.biases.view(np.uint32), b.view(np.uint32)), key
            codes = (m.weights.astype(np.uint64)[:, None] >> (4 * np.arange(8, dtype=np.uint64))) & 15
            deq = (codes.reshape(rows, cols // 32, 32) * m.scales.reshape(rows, -1, 1).astype(np.float64)
                   + m.biases.reshape(rows, -1, 1))
            orig = z[f"{key}/f16"].view(np.float16).astype(np.float64).reshape(rows, cols // 32, 32)
            # Round to the nearest code (half a step), plus the rounding of the
            # stored scale (15 steps) and bias to 11 (F16) or 8 (BF16) bits.
            ulp = 2.0 ** (-10 if kind == "F16" else -7)
            tol = (0.5 * m.scales.reshape(rows, -1, 1) + 16 * ulp * m.scales.reshape(rows, -1, 1)
                   + ulp * np.abs(m.biases.reshape(rows, -1, 1)) + 1e-7)
            assert np.all(np.abs(deq - orig) <= tol), key


def test_dense_fixture_checkpoint_keeps_f16_bits(tmp_path):
    """The original tiny checkpoint's F16 matrices (no quantisation) read back
    bit for bit as dense matrices."""
    z = _fixture()
    names = _matrix_names(z)
    tensors = [(key.replace("/", ".") + ".weight", "F16", [int(v) for v in z[f"{key}/shape"]],
                z[f"{key}/f16"].tobytes()) for key in names]
    write_config(tmp_path)
    write_tensor_file(tmp_path / "model.safetensors", tensors)
    with qmr.Checkpoint(tmp_path) as cp:
        for key in names:
            d = cp.matrix(key.replace("/", "."))
            assert isinstance(d, qmr.DenseData)
            assert np.array_equal(d.values, z[f"{key}/f16"]), key


# ------------------------------------------------------------- conversions


def _dense_round_trip(tmp_path, dtype: str, payload: bytes, n: int) -> np.ndarray:
    write_config(tmp_path)
    write_tensor_file(tmp_path / "model.safetensors", [("model.w.weight", dtype, [1, n], payload)])
    with qmr.Checkpoint(tmp_path) as cp:
        return cp.matrix("model.w").values


def test_dense_f32_converts_to_f16_round_to_nearest_even(tmp_path):
    """Every binade of binary16 (subnormals included), exact ties and the
    largest finite value: identical to numpy's IEEE conversion."""
    rng = np.random.default_rng(5)
    e = rng.uniform(-27, 16, 20000)
    v = (np.sign(rng.standard_normal(e.size)) * 2.0 ** e).astype(np.float32)
    v = v[np.abs(v) <= 65504]
    h = np.arange(0, 0x7BFF, 7, dtype=np.uint16).view(np.float16).astype(np.float32)
    ties = ((h[:-1].astype(np.float64) + h[1:]) / 2).astype(np.float32)  # halfway points are f32-exact
    special = np.array([0.0, -0.0, 65504.0, -65504.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                        2.0 ** -14, 2.0 ** -14 - 2.0 ** -25], np.float32)
    allv = np.concatenate([v, ties, special])
    got = _dense_round_trip(tmp_path, "F32", allv.tobytes(), allv.size)
    assert np.array_equal(got, allv.astype(np.float16).view(np.uint16))


def test_dense_bf16_converts_to_f16(tmp_path):
    rng = np.random.default_rng(6)
    bits = rng.integers(0, 1 << 16, 30000).astype(np.uint16)
    vals = (bits.astype(np.uint32) << 16).view(np.float32)
    keep = np.isfinite(vals) & (np.abs(vals) <= 65504)
    got = _dense_round_trip(tmp_path, "BF16", bits[keep].tobytes(), int(keep.sum()))
    assert np.array_equal(got, vals[keep].astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("value", [65520.0, -1e6, float("inf"), float("nan")])
def test_dense_values_beyond_f16_are_rejected(tmp_path, value):
    write_config(tmp_path)
    write_tensor_file(tmp_path / "model.safetensors", [("model.w.weight", "F32", [1, 2], f32(1.0, value))])
    with qmr.Checkpoint(tmp_path) as cp:
        with pytest.raises(qmr.QmrError, match="exceeds F16 range"):
            cp.matrix("model.w")


# ----------------------------------------------- quantisation and lookups


def _packed(tmp_path, quant, words=(0x76543210,), meta="F16", scales=(0x3800,), biases=(0xBC00,),
            name="model.layers.0.mlp.gate_proj", wshape=(1, 1), mshape=(1, 1), **cfg):
    write_config(tmp_path, **({"quantization": quant} if quant is not None else {}), **cfg)
    write_tensor_file(tmp_path / "model.safetensors", [
        (f"{name}.weight", "U32", list(wshape), u32(*words)),
        (f"{name}.scales", meta, list(mshape), u16(*scales) if meta != "F32" else f32(*scales)),
        (f"{name}.biases", meta, list(mshape), u16(*biases) if meta != "F32" else f32(*biases)),
    ])
    return qmr.Checkpoint(tmp_path)


def test_quantization_config_alias_and_disabled_override(tmp_path):
    cp = _packed(tmp_path, None, quantization_config={"bits": 4, "group_size": 8})
    assert cp.matrix_info("model.layers.0.mlp.gate_proj").bits == 4
    cp.close()
    cp = _packed(tmp_path, {"bits": 4, "group_size": 8, "model.layers.0.mlp.gate_proj": False})
    with pytest.raises(qmr.QmrError, match="packed matrix lacks quantization metadata"):
        cp.matrix_info("model.layers.0.mlp.gate_proj")
    cp.close()
    cp = _packed(tmp_path, None)
    with pytest.raises(qmr.QmrError, match="packed matrix lacks quantization metadata"):
        cp.matrix("model.layers.0.mlp.gate_proj")


@pytest.mark.parametrize("quant,needle", [
    ({"bits": 3, "group_size": 8}, "unsupported quantization bit width 3"),
    ({"bits": 4, "group_size": 12}, "invalid quantization group size"),
    ({"bits": 4}, "missing quantization group size"),
    ({"bits": 4, "group_size": 8, "mode": "mxfp4"}, "unsupported quantization mode mxfp4"),
    ({"bits": 4, "group_size": 8, "model.x": 3}, "invalid quantization entry model.x"),
    ({"bits": 4, "group_size": 8, "language_model.model.x": True, "model.x": False},
     "duplicate quantization entry model.x"),
])
def test_invalid_quantization_metadata_is_rejected(tmp_path, quant, needle):
    write_config(tmp_path, quantization=quant)
    write_tensor_file(tmp_path / "model.safetensors", [("model.norm.weight", "F32", [1], f32(0.0))])
    rejected(tmp_path, needle)


def test_packed_shape_and_metadata_checks(tmp_path):
    q = {"bits": 4, "group_size": 16}  # two words per group
    cp = _packed(tmp_path, q, words=(1, 2, 3), wshape=(1, 3))
    with pytest.raises(qmr.QmrError, match="packed width not divisible by group width"):
        cp.matrix_info("model.layers.0.mlp.gate_proj")
    cp.close()
    cp = _packed(tmp_path, q, words=(1, 2), wshape=(1, 2), scales=(0x3800, 0x3800), biases=(0, 0),
                 mshape=(1, 2))
    with pytest.raises(qmr.QmrError, match="scales shape mismatch"):
        cp.matrix_info("model.layers.0.mlp.gate_proj")
    cp.close()
    cp = _packed(tmp_path, {"bits": 4, "group_size": 8}, scales=(0x7C00,))  # +inf in F16
    assert cp.matrix_info("model.layers.0.mlp.gate_proj").packed
    with pytest.raises(qmr.QmrError, match="scales contains non-finite values"):
        cp.matrix("model.layers.0.mlp.gate_proj")
    cp.close()
    cp = _packed(tmp_path, {"bits": 8, "group_size": 4}, meta="F32", scales=(0.25,), biases=(-32.0,))
    m = cp.matrix("model.layers.0.mlp.gate_proj")
    assert (m.rows, m.cols, m.bits, m.group_size) == (1, 4, 8, 4)
    assert m.scales.tolist() == [0.25] and m.biases.tolist() == [-32.0]


def test_tied_lm_head(tmp_path):
    """Checkpoint::tensor / contains (src/weights.rs:389-410): with
    tie_word_embeddings a missing lm_head.weight is the embedding. A packed
    tied head still needs lm_head.scales, exactly as in the reference."""
    write_config(tmp_path, text_config={"tie_word_embeddings": True})
    write_tensor_file(tmp_path / "model.safetensors", [
        ("language_model.model.embed_tokens.weight", "F16", [2, 2], u16(0x3C00, 0x4000, 0x4200, 0x4400))])
    with qmr.Checkpoint(tmp_path) as cp:
        assert cp.contains("lm_head") and cp.contains("model.embed_tokens")
        assert cp.matrix("lm_head").values.tolist() == [0x3C00, 0x4000, 0x4200, 0x4400]
    write_config(tmp_path)
    with qmr.Checkpoint(tmp_path) as cp:
        assert not cp.contains("lm_head")
        with pytest.raises(qmr.QmrError, match="missing tensor lm_head.weight"):
            cp.matrix_info("lm_head")
    write_config(tmp_path, tie_word_embeddings=True, quantization={"bits": 4, "group_size": 8})
    write_tensor_file(tmp_path / "model.safetensors", [
        ("model.embed_tokens.weight", "U32", [1, 1], u32(5)),
        ("model.embed_tokens.scales", "F16", [1, 1], u16(0x3C00)),
        ("model.embed_tokens.biases", "F16", [1, 1], u16(0)),
    ])
    with qmr.Checkpoint(tmp_path) as cp:
        assert cp.matrix_info("model.embed_tokens").packed
        with pytest.raises(qmr.QmrError, match="missing tensor lm_head.scales"):
            cp.matrix_info("lm_head")


# ----------------------------------------------- safetensors validation


def _one(tmp_path, header: dict, data: bytes):
    write_config(tmp_path)
    write_raw(tmp_path / "model.safetensors", json.dumps(header).encode(), data)


@pytest.mark.parametrize("header,data,needle", [
    ({"a.weight": {"dtype": "F32", "shape": [0], "data_offsets": [0, 0]}}, b"", "zero tensor dimension"),
    ({"a.weight": {"dtype": "C64", "shape": [1], "data_offsets": [0, 8]}}, bytes(8), "unsupported dtype C64"),
    ({"a.weight": {"shape": [1], "data_offsets": [0, 4]}}, bytes(4), "missing dtype"),
    ({"a.weight": {"dtype": "F32", "data_offsets": [0, 4]}}, bytes(4), "missing shape"),
    ({"a.weight": {"dtype": "F32", "shape": [1]}}, bytes(4), "missing data offsets"),
    ({"a.weight": {"dtype": "F32", "shape": [1], "data_offsets": [0]}}, bytes(4), "invalid data offsets"),
    ({"a.weight": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}, bytes(4), "invalid tensor dimension"),
    ({"a.weight": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, bytes(4), "tensor exceeds file"),
    ({"a.weight": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},
      "b.weight": {"dtype": "F32", "shape": [1], "data_offsets": [2, 6]}}, bytes(8), "overlap or leave holes"),
    ({"a.weight": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, bytes(8), "overlap or leave holes"),
    ({"__metadata__": ["x"]}, b"", "invalid safetensors metadata"),
    ([1, 2], b"", "safetensors header is not an object"),
    ({"a.weight": {"dtype": "U8", "shape": [3], "data_offsets": [0, 3]},
      "model.a.weight": {"dtype": "U8", "shape": [1], "data_offsets": [3, 4]},
      "language_model.model.a.weight": {"dtype": "U8", "shape": [1], "data_offsets": [4, 5]}},
     bytes(5), "duplicate canonical tensor model.a.weight"),
])
def test_malformed_safetensors_are_rejected(tmp_path, header, data, needle):
    _one(tmp_path, header, data)
    rejected(tmp_path, needle)


def test_header_bounds(tmp_path):
    write_config(tmp_path)
    (tmp_path / "model.safetensors").write_bytes(b"\x01\x02")
    rejected(tmp_path, "safetensors header truncated")
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", 100_000_001) + b"{}")
    rejected(tmp_path, "safetensors header exceeds 100 MB")
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", 50) + b"{}")
    rejected(tmp_path, "safetensors header truncated")
    write_raw(tmp_path / "model.safetensors", b'{"a.weight": {"dtype": "F32",}}')
    rejected(tmp_path, "invalid safetensors JSON header")
    write_raw(tmp_path / "model.safetensors", b"{}   ")
    with qmr.Checkpoint(tmp_path) as cp:
        assert len(cp) == 0


def test_shard_discovery(tmp_path):
    write_config(tmp_path)
    rejected(tmp_path, "expected one safetensors file or an index")
    write_tensor_file(tmp_path / "a.safetensors", [("model.x.weight", "F16", [1, 1], u16(0x3C00))])
    write_tensor_file(tmp_path / "b.safetensors", [("model.y.weight", "F16", [1, 1], u16(0x3C00))])
    rejected(tmp_path, "expected one safetensors file or an index")
    index = tmp_path / "model.safetensors.index.json"
    index.write_text(json.dumps({"weight_map": {"model.x.weight": "a.safetensors",
                                                "model.y.weight": "b.safetensors"}}))
    with qmr.Checkpoint(tmp_path) as cp:
        assert len(cp) == 2 and cp.contains("model.x") and cp.contains("model.y.weight")
    index.write_text(json.dumps({"weight_map": {"model.x.weight": "a.safetensors",
                                                "model.y.weight": "b.safetensors",
                                                "model.z.weight": "b.safetensors"}}))
    rejected(tmp_path, "index names missing from shards")
    index.write_text(json.dumps({"weight_map": {}}))
    rejected(tmp_path, "empty safetensors index")
    index.write_text(json.dumps({"weight_map": {"model.x.weight": "a.bin"}}))
    rejected(tmp_path, "unsafe shard filename a.bin")
    os.remove(index)
    os.remove(tmp_path / "b.safetensors")
    os.remove(tmp_path / "config.json")
    with pytest.raises(qmr.QmrError, match="config.json"):
        qmr.Checkpoint(tmp_path)


def test_symlinked_shard_outside_the_directory_is_rejected(tmp_path):
    outside = tmp_path / "outside"
    ck = tmp_path / "ck"
    outside.mkdir()
    ck.mkdir()
    write_tensor_file(outside / "x.safetensors", [("model.x.weight", "F16", [1, 1], u16(0x3C00))])
    write_config(ck)
    os.symlink(outside / "x.safetensors", ck / "model.safetensors")
    rejected(ck, "safetensors shard escapes checkpoint directory")


# ------------------------------------------------ malformed input robustness

from hypothesis import HealthCheck, given, settings  # noqa: E402
from hypothesis import strategies as st  # noqa: E402

_GOOD_HEADER = json.dumps({
    "__metadata__": {"format": "mlx"},
    "model.a.weight": {"dtype": "U32", "shape": [2, 1], "data_offsets": [0, 8]},
    "model.a.scales": {"dtype": "BF16", "shape": [2, 1], "data_offsets": [8, 12]},
    "model.a.biases": {"dtype": "BF16", "shape": [2, 1], "data_offsets": [12, 16]},
}).encode()


@settings(max_examples=300, deadline=None, suppress_health_check=[HealthCheck.function_scoped_fixture])
@given(st.binary(max_size=200), st.integers(0, len(_GOOD_HEADER)), st.integers(0, 40))
def test_random_and_mutated_headers_fail_cleanly(tmp_path, noise, cut, data_len):
    """Random bytes spliced into a valid header, truncated headers and data
    sections of any length: opening either succeeds or raises QmrError, and
    a checkpoint that opens answers matrix queries the same way."""
    write_config(tmp_path, quantization={"bits": 4, "group_size": 8})
    header = _GOOD_HEADER[:cut] + noise + _GOOD_HEADER[cut:]
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", len(header)) + header + bytes(data_len))
    try:
        cp = qmr.Checkpoint(tmp_path)
    except qmr.QmrError:
        return
    with cp:
        for name in ("model.a", "model.b", "lm_head"):
            try:
                cp.matrix(name)
            except qmr.QmrError:
                pass


@settings(max_examples=200, deadline=None, suppress_health_check=[HealthCheck.function_scoped_fixture])
@given(st.recursive(st.none() | st.booleans() | st.integers(-2**70, 2**70) | st.floats(allow_nan=False)
                    | st.text(max_size=8),
                    lambda inner: st.lists(inner, max_size=4) | st.dictionaries(st.text(max_size=6), inner,
                                                                                max_size=4),
                    max_leaves=20))
def test_arbitrary_json_values_as_headers_fail_cleanly(tmp_path, value):
    write_config(tmp_path)
    header = json.dumps(value).encode()
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", len(header)) + header)
    try:
        qmr.Checkpoint(tmp_path).close()
    except qmr.QmrError:
        pass

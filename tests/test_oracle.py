"""Pins the CPU oracle (oracle/qmr_oracle.c) before anything is checked
against it. Every oracle function is checked by something it does not
share code with:
  - the reference's own known answers (src/weights.rs:816-870,
    src/gpu.rs:1637-1657,1699-1732, tests/batch_matrix.rs:176-232,358-381,
    src/gpu/metadata.rs:24-58);
  - the reference's genuine MLX fixture bytes (tests/fixtures/tiny-q4 and
    tiny-bf16, extracted to tests/golden/mlx_fixtures.npz), re-derived from
    the dense F16 originals with the fixture quantiser the reference
    published (scripts/make_fixture.py:197-210, 262-290);
  - numpy's IEEE half conversion (all 65536 patterns) and BLAS;
  - closed forms: one-hot columns, row sums read from the little-endian
    byte view, linearity, exact power-of-two scaling, batch stacking.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def f16bits(values):
    return np.asarray(values, dtype=np.float16).view(np.uint16)


# ---------------------------------------------------------------- KATs


def test_nibble_order_and_f16_metadata_kat():
    # src/weights.rs:816-870: 0x76543210 with F16 scale 0x3800 (0.5), bias 0xbc00 (-1).
    w = np.array([0x76543210], np.uint32)
    s = np.array([0x3800], np.uint16)
    b = np.array([0xBC00], np.uint16)
    got = oracle.dequant_row(w, s, b, "f16", 0, 8, 4, 8)
    assert got.tolist() == [-1.0, -0.5, 0.0, 0.5, 1.0, 1.5, 2.0, 2.5]
    assert oracle.f16_to_f32(0x3800) == 0.5 and oracle.f16_to_f32(0xBC00) == -1.0


def test_q4_little_nibbles_and_bias_kat():
    # src/gpu.rs:1637-1657 -> [48, 14].
    w = np.array([0x76543210, 0xFEDCBA98], np.uint32)
    s = np.array([2.0, 0.5], np.float32)
    b = np.array([-1.0, -4.0], np.float32)
    y = oracle.matmul_f64(w, s, b, "f32", np.ones(8, np.float32), 2, 8, 4, 8)
    assert y.tolist() == [48.0, 14.0]


def test_q8_matvec_and_embedding_kat():
    # src/gpu.rs:1714-1730 -> [693, 30]; embedding row 0 -> [-1, -0.5, 63, 126.5].
    w = np.array([0xFF800100, 0x04030201], np.uint32)
    s = np.array([0.5, 2.0], np.float32)
    b = np.array([-1.0, -3.0], np.float32)
    x = np.array([1, 2, 3, 4], np.float32)
    assert oracle.matmul_f64(w, s, b, "f32", x, 2, 4, 8, 4).tolist() == [693.0, 30.0]
    assert oracle.dequant_row(w, s, b, "f32", 0, 4, 8, 4).tolist() == [-1.0, -0.5, 63.0, 126.5]


def test_stream_and_offset_kats():
    # tests/batch_matrix.rs:358-381: four rows of 0x76543210, s=1, b=0, x=1 -> 1792.
    w = np.full(4 * 512 // 8, 0x76543210, np.uint32)
    one, zero = np.ones(32, np.float32), np.zeros(32, np.float32)
    y = oracle.matmul_f64(w, one, zero, "f32", np.ones(512, np.float32), 4, 512, 4, 64)
    assert y.tolist() == [1792.0] * 4
    # tests/batch_matrix.rs:223-232: zero codes, s=b=1, x=2 -> 1024.
    w0 = np.zeros(4 * 512 // 8, np.uint32)
    y = oracle.matmul_f64(w0, one, one, "f32", np.full(512, 2.0, np.float32), 4, 512, 4, 64)
    assert y.tolist() == [1024.0] * 4


def test_bf16_pack_patterns_round_trip_and_rejections():
    # src/gpu/metadata.rs:24-45 and :47-58.
    patterns = np.array([0x00000000, 0x80000000, 0x3FC00000, 0xC0200000, 0x00010000,
                         0x80010000, 0x00800000, 0x7F7F0000], np.uint32)
    packed = oracle.pack_bf16_exact(patterns.view(np.float32))
    assert packed is not None
    assert ((packed.astype(np.uint32) << 16) == patterns).all()
    for h, bits in zip(packed, patterns):
        assert np.float32(oracle.bf16_to_f32(int(h))).view(np.uint32) == bits
    for bad in (0.1, np.uint32(1).view(np.float32), np.inf, -np.inf, np.nan):
        assert oracle.pack_bf16_exact(np.array([1.0, bad, -0.0], np.float32)) is None


def test_f16_decoding_matches_ieee_for_every_pattern():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    assert (got[~nan].view(np.uint32) == want[~nan].view(np.uint32)).all()


# ------------------------------------------------- genuine MLX fixture bytes


def _fixture():
    return np.load(GOLDEN / "mlx_fixtures.npz")


def _matrices(z):
    return sorted({k.rsplit("/", 1)[0] for k in z.files if k.endswith("/shape")})


def _quantise_like_fixture(orig_f16_bits, rows, cols, kind):
    """scripts/make_fixture.py:197-210 (F16 metadata) and 279-290 (BF16):
    per 32-column group, scale = R((max-min)/15), bias = R(min),
    q = clamp(round_half_even((v - bias)/scale), 0, 15)."""
    v = orig_f16_bits.view(np.float16).astype(np.float64).reshape(rows, cols // 32, 32)
    lo, hi = v.min(axis=2), v.max(axis=2)
    if kind == "f16":
        scale = ((hi - lo) / 15).astype(np.float16).astype(np.float64)
        bias = lo.astype(np.float16).astype(np.float64)
        s_bits = scale.astype(np.float16).view(np.uint16)
        b_bits = bias.astype(np.float16).view(np.uint16)
    else:
        def bf16(x):
            bits = x.astype(np.float32).view(np.uint32).astype(np.uint64)
            r = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint32)
            return r.astype(np.uint16), (r << 16).view(np.float32).astype(np.float64)
        s_bits, scale = bf16((hi - lo) / 15)
        b_bits, bias = bf16(lo)
    q = np.clip(np.round((v - bias[..., None]) / scale[..., None]), 0, 15).astype(np.uint64)
    q8 = q.reshape(rows, cols // 8, 8)
    words = np.zeros((rows, cols // 8), np.uint64)
    for i in range(8):
        words |= q8[..., i] << np.uint64(4 * i)
    deq = (q * scale[..., None] + bias[..., None]).reshape(rows, cols)
    return words.astype(np.uint32).ravel(), s_bits.ravel(), b_bits.ravel(), q.reshape(rows, cols), deq


@pytest.mark.parametrize("tag,kind", [("q4f16", "f16"), ("q4bf16", "bf16")])
def test_fixture_bytes_match_published_quantiser_and_oracle_dequant(tag, kind):
    z = _fixture()
    names = _matrices(z)
    assert len(names) == 33  # the reference counts 33 compacted matrices (tests/bf16_inference.rs)
    for key in names:
        rows, cols = (int(v) for v in z[f"{key}/shape"])
        w, s, b = z[f"{key}/{tag}/w"], z[f"{key}/{tag}/s"], z[f"{key}/{tag}/b"]
        words, s_bits, b_bits, q, deq = _quantise_like_fixture(z[f"{key}/f16"], rows, cols, kind)
        assert np.array_equal(w, words), key
        assert np.array_equal(s, s_bits) and np.array_equal(b, b_bits), key
        # Oracle unpack and metadata decoding of the genuine bytes.
        for r in range(rows):
            got = oracle.dequant_row(w, s, b, kind, r, cols, 4, 32)
            assert np.array_equal(got, deq[r].astype(np.float32)), (key, r)
        assert all(oracle.code(w, cols, 4, r, c) == q[r, c]
                   for r in (0, rows - 1) for c in range(cols))


def test_fixture_matvec_agrees_with_blas_on_dequantised_weights():
    z = _fixture()
    rng = np.random.default_rng(7)
    for key in _matrices(z):
        rows, cols = (int(v) for v in z[f"{key}/shape"])
        w, s, b = z[f"{key}/q4bf16/w"], z[f"{key}/q4bf16/s"], z[f"{key}/q4bf16/b"]
        _, _, _, _, deq = _quantise_like_fixture(z[f"{key}/f16"], rows, cols, "bf16")
        x = rng.standard_normal((3, cols)).astype(np.float32)
        y = oracle.matmul_f64(w, s, b, "bf16", x, rows, cols, 4, 32, batch=3)
        want = (x.astype(np.float64) @ deq.T).ravel()
        np.testing.assert_allclose(y, want, rtol=1e-12, atol=1e-12)


# ----------------------------------------------------------- closed forms


def _random_q4(rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 2**32, size=rows * cols // 8, dtype=np.uint32)
    return w


def _codes_from_bytes(w, rows, cols):
    """Codes read through the little-endian byte view: byte k holds column
    2k in its low nibble and 2k+1 in its high nibble."""
    by = w.view(np.uint8).reshape(rows, cols // 2)
    out = np.empty((rows, cols), np.int64)
    out[:, 0::2] = by & 15
    out[:, 1::2] = by >> 4
    return out


def test_one_hot_columns_and_row_sums():
    rows, cols, group = 5, 256, 64
    w = _random_q4(rows, cols, 1)
    codes = _codes_from_bytes(w, rows, cols)
    ones = np.ones(rows * cols // group, np.float32)
    zeros = np.zeros_like(ones)
    for c in (0, 1, 7, 8, 63, 64, 255):
        x = np.zeros(cols, np.float32)
        x[c] = 1.0
        y = oracle.matmul_f64(w, ones, zeros, "f32", x, rows, cols, 4, group)
        assert y.tolist() == codes[:, c].astype(float).tolist()
    y = oracle.matmul_f64(w, ones, zeros, "f32", np.ones(cols, np.float32), rows, cols, 4, group)
    assert y.tolist() == codes.sum(axis=1).astype(float).tolist()
    # Bias alone: x = 1, s = 0, b = per-group constants -> group * sum(b).
    bvals = np.arange(rows * cols // group, dtype=np.float32) - 3
    y = oracle.matmul_f64(w, zeros, bvals, "f32", np.ones(cols, np.float32), rows, cols, 4, group)
    assert y.tolist() == (group * bvals.reshape(rows, -1).sum(axis=1)).astype(float).tolist()


def test_q8_codes_are_little_endian_bytes():
    rows, cols, group = 3, 128, 32
    rng = np.random.default_rng(2)
    w = rng.integers(0, 2**32, size=rows * cols // 4, dtype=np.uint32)
    codes = w.view(np.uint8).reshape(rows, cols).astype(np.int64)
    ones = np.ones(rows * cols // group, np.float32)
    zeros = np.zeros_like(ones)
    for c in (0, 1, 2, 3, 4, 127):
        x = np.zeros(cols, np.float32)
        x[c] = 1.0
        assert oracle.matmul_f64(w, ones, zeros, "f32", x, rows, cols, 8, group).tolist() == \
            codes[:, c].astype(float).tolist()


def test_linearity_scaling_batch_and_thread_invariance():
    rows, cols, group = 9, 512, 64
    w = _random_q4(rows, cols, 3)
    rng = np.random.default_rng(4)
    s = rng.uniform(0.002, 0.02, rows * cols // group).astype(np.float32)
    b = (-8 * s + rng.normal(0, 1e-3, s.size)).astype(np.float32)
    x1 = rng.standard_normal(cols).astype(np.float32)
    x2 = rng.standard_normal(cols).astype(np.float32)
    f = lambda x, **k: oracle.matmul_f64(w, s, b, "f32", x, rows, cols, 4, group, **k)
    np.testing.assert_allclose(f(x1 + x2), f(x1) + f(x2), rtol=1e-6, atol=1e-6)
    assert np.array_equal(f(np.float32(4.0) * x1), 4.0 * f(x1))  # exact power-of-two scaling
    xb = np.stack([x1, x2, -x1])
    yb = oracle.matmul_f64(w, s, b, "f32", xb, rows, cols, 4, group, batch=3)
    assert np.array_equal(yb, np.concatenate([f(x1), f(x2), f(-x1)]))
    assert np.array_equal(f(x1, threads=4), f(x1, threads=1))
    y32 = oracle.matmul_f32(w, s, b, "f32", x1, rows, cols, 4, group)
    np.testing.assert_allclose(y32, f(x1), rtol=1e-4, atol=1e-4)


def test_invalid_shapes_are_rejected():
    w = np.zeros(8, np.uint32)
    m = np.zeros(8, np.float32)
    for rows, cols, bits, group in [(2, 7, 4, 8), (2, 8, 3, 8), (2, 8, 4, 0), (0, 8, 4, 8)]:
        with pytest.raises(ValueError):
            oracle.matmul_f64(w, m, m, "f32", np.zeros(max(cols, 1), np.float32), rows, cols,
                              bits, group)


def test_dense_f16_oracle_matches_blas():
    rng = np.random.default_rng(5)
    rows, cols = 7, 37
    w16 = f16bits(((rng.integers(0, 41, rows * cols)) - 20) / 32.0)
    x = rng.standard_normal((4, cols)).astype(np.float32)
    y = oracle.dense_f16_f64(w16, x, rows, cols, 4)
    want = (x.astype(np.float64) @ w16.view(np.float16).astype(np.float64).reshape(rows, cols).T)
    np.testing.assert_allclose(y, want.ravel(), rtol=1e-13, atol=1e-13)


# ------------------------------------------------------ config 0 golden


def test_config0_golden_vector():
    """Regression pin of the generator + oracle on BASELINE config 0."""
    import qmr.synth as synth

    z = np.load(GOLDEN / "config0.npz")
    m = synth.q4_bf16_matrix(1024, 1024, int(z["seed"]), tag="config0")
    x = synth.activations(1024, 1, int(z["seed"]), tag="config0")
    assert np.array_equal(m.w[:16], z["w_head"]) and np.array_equal(m.s[:16], z["s_head"])
    assert np.array_equal(m.b[:16], z["b_head"]) and np.array_equal(x.ravel()[:16], z["x_head"])
    y = oracle.matmul_f64(m.w, m.s, m.b, "bf16", x, 1024, 1024, 4, 64)
    assert np.array_equal(y, z["y64"])


# ------------------------------------- the decoder layer's elementwise steps


def test_rms_norm_swiglu_and_add_kats():
    """src/gpu.rs:1785-1791 (rms_norm), 1822-1825 (swiglu, add)."""
    eps = float(np.float32(1e-6))
    d = np.sqrt(12.5 + eps)
    np.testing.assert_allclose(oracle.rms_norm_f64([3.0, 4.0], [2.0, 1.0], eps), [6 / d, 4 / d], rtol=1e-15)
    np.testing.assert_allclose(oracle.swiglu_f64([0.0, 1.0], [3.0, 4.0]), [0.0, 4 / (1 + np.exp(-1.0))],
                               rtol=1e-15)
    # The Q4 known answer (src/gpu.rs:1637-1657) with a residual: [48, 14] + [0, 1].
    w = np.array([0x76543210, 0xFEDCBA98], np.uint32)
    y = oracle.matmul_add_f64(w, np.array([2.0, 0.5], np.float32), np.array([-1.0, -4.0], np.float32), "f32",
                              np.ones(8, np.float32), [0.0, 1.0], 2, 8, 4, 8)
    assert y.tolist() == [48.0, 15.0]


def test_rms_norm_and_silu_identities():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 257))
    w = rng.uniform(0.5, 2.0, 257)
    # Scale invariance as eps -> 0, and unit RMS for unit weights.
    np.testing.assert_allclose(oracle.rms_norm_f64(7.5 * x, w, 1e-300), oracle.rms_norm_f64(x, w, 1e-300),
                               rtol=1e-13)
    y = oracle.rms_norm_f64(x, np.ones(257), 1e-300)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=1)), 1.0, rtol=1e-13)
    # eps enters under the root: mean(y^2) = m / (m + eps) for unit weights.
    m = np.mean(x * x, axis=1)
    y = oracle.rms_norm_f64(x, np.ones(257), 0.25)
    np.testing.assert_allclose(np.mean(y * y, axis=1), m / (m + 0.25), rtol=1e-13)
    # silu(g) - silu(-g) = g; silu(0) = 0; silu(g) -> g for large g.
    g = rng.standard_normal(1000) * 6
    one = np.ones_like(g)
    np.testing.assert_allclose(oracle.swiglu_f64(g, one) - oracle.swiglu_f64(-g, one), g, rtol=1e-12, atol=1e-15)
    assert oracle.swiglu_f64([0.0], [5.0]).tolist() == [0.0]
    np.testing.assert_allclose(oracle.swiglu_f64([40.0], [1.0]), [40.0], rtol=1e-15)


def test_mlp_oracle_matches_a_scalar_brute_force():
    """mlp_gate_up_f64 against loops over the reference's per-weight formula
    (tests/quantized.rs:39-51) and the elementwise kernels, on a 5x64 Q4/g32
    case with two RHS."""
    import math

    rng = np.random.default_rng(11)
    rows, cols, group, batch, eps = 5, 64, 32, 2, 1e-5
    mats = []
    for _ in range(2):
        w = rng.integers(0, 2**32, rows * cols // 8, dtype=np.uint64).astype(np.uint32)
        s = rng.uniform(0.01, 0.1, rows * cols // group).astype(np.float32)
        b = (-8 * s + rng.normal(0, 1e-3, s.size)).astype(np.float32)
        mats.append((w, s, b))
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    got = oracle.mlp_gate_up_f64(mats[0], mats[1], "f32", x, nw, eps, rows, cols, 4, group, batch)

    def product(m, v, r):
        w, s, b = m
        acc = 0.0
        for c in range(cols):
            q = (int(w[r * (cols // 8) + c // 8]) >> (4 * (c % 8))) & 15
            gi = r * (cols // group) + c // group
            acc += (q * float(s[gi]) + float(b[gi])) * float(v[c])
        return acc

    for t in range(batch):
        ms = sum(float(v) * float(v) for v in x[t]) / cols
        inv = 1.0 / math.sqrt(ms + eps)
        n = [float(np.float32(float(x[t, c]) * inv * float(nw[c]))) for c in range(cols)]
        for r in range(rows):
            g, u = product(mats[0], n, r), product(mats[1], n, r)
            want = g / (1.0 + math.exp(-g)) * u
            assert abs(got[t * rows + r] - want) <= 1e-12 * max(1.0, abs(want)), (t, r)


def test_dequant_row_rounds_product_then_sum_for_fp32_metadata():
    """kernels/qwen.metal:40-47 writes float(q) * s[gi] + b[gi]: with FP32
    metadata the product (up to 8 + 24 significant bits) is rounded before the
    sum. The oracle's row equals numpy's float32 multiply then add (each op
    rounded) for every element, and differs from the single-rounding
    RN32(q*s + b) on some, so the check tells the two apart."""
    rng = np.random.default_rng(17)
    rows, cols, bits, group = 3, 4096, 8, 32
    w = rng.integers(0, 2**32, rows * cols * bits // 32, dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.001, 0.02, rows * cols // group).astype(np.float32)
    b = rng.uniform(-1.0, 1.0, rows * cols // group).astype(np.float32)
    shifts = (np.arange(cols) % (32 // bits)) * bits
    fused_differs = 0
    for r in range(rows):
        words = w.reshape(rows, -1)[r][np.arange(cols) // (32 // bits)]
        q = ((words >> shifts.astype(np.uint32)) & ((1 << bits) - 1)).astype(np.float32)
        sg = s.reshape(rows, -1)[r][np.arange(cols) // group]
        bg = b.reshape(rows, -1)[r][np.arange(cols) // group]
        want = (q * sg) + bg  # float32 ops, each rounded
        fused = (q.astype(np.float64) * sg.astype(np.float64) + bg.astype(np.float64)).astype(np.float32)
        got = oracle.dequant_row(w, s, b, "f32", r, cols, bits, group)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), r
        fused_differs += int(np.count_nonzero(fused != want))
    assert fused_differs > 0

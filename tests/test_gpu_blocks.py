"""Small-block (B = 1..4) parity on the GPU, restating tests/batch_matrix.rs:
  :17-105   all batches, formats, tails, non-zero 4-byte offsets, guards
  :108-174  dense F16 blocks with offsets and guard values
  :176-232  offset dispatch, bounds and alias rejection, scalar offset KAT
  :236-354  aligned Q4 blocks vs FP64 and vs sequential GEMVs; the
            Legacy / Shared / MLP-R2 schedules agree bit for bit
  :358-381  stream fallback KAT (weights at a 4-byte offset)
  :386-636  full 17408x5120 and 5120x17408 B=3 BF16 with input/output
            guards, Legacy vs R2 bit identity, 32 sampled rows vs FP64
"""
import numpy as np
import pytest

import oracle
import qmr
from helpers import assert_close_ref, assert_gate

pytestmark = pytest.mark.gpu


def block_close(got, want, what):
    # tests/batch_matrix.rs:5-14: 4e-4 + 3e-5*|want|.
    assert_close_ref(got, want, 4e-4, 3e-5, what)


def test_affine_blocks_share_weights_for_all_batches_formats_tails_and_offsets(gpu):
    for bits in (4, 8):
        for group in (32, 64, 128):
            for rows, cols in ((1, group), (3, 3 * group), (7, 512), (20, 5120)):
                pack = 32 // bits
                i = np.arange(rows * cols // pack, dtype=np.uint64)
                w = ((i * 0x9E3779B9 + 0x1478ABCF) & 0xFFFFFFFF).astype(np.uint32)
                n = rows * cols // group
                k = np.arange(n)
                s = ((1 + k % 11) * 0.001953125).astype(np.float32)
                b = ((k % 9) * 0.00390625 - 0.0625).astype(np.float32)
                x = ((((np.arange(4 * cols) * 13) % 101) - 50) / 50).astype(np.float32)
                for bf16 in (False, True):
                    meta = (s.view(np.uint32) >> 16).astype(np.uint16) if bf16 else s
                    bmeta = (b.view(np.uint32) >> 16).astype(np.uint16) if bf16 else b
                    kind = "bf16" if bf16 else "f32"
                    want = oracle.matmul_f64(w, meta, bmeta, kind, x, rows, cols, bits, group, 4)
                    pad = lambda a: np.concatenate([np.zeros(4, np.uint8), np.frombuffer(a.tobytes(), np.uint8)])
                    wb = gpu.upload_bytes(pad(w))
                    sb = gpu.upload_bytes(pad(meta))
                    bb = gpu.upload_bytes(pad(bmeta))
                    xb = gpu.upload_f32(np.concatenate([[99.0], x, [99.0]]))
                    name = "matmul_affine_bf16" if bf16 else "matmul_affine"
                    for batch in range(1, 5):
                        yb = gpu.upload_f32(np.full(batch * rows + 2, 12345.0))
                        gpu.dispatch(name, [wb, sb, bb, xb, yb], [rows, cols, bits, group, batch],
                                     offsets=[4] * 5)
                        got = gpu.read_f32(yb, batch * rows + 2)
                        assert got[0] == 12345.0 and got[batch * rows + 1] == 12345.0
                        # Token-major: the first `batch` RHS of the oracle's 4.
                        block_close(got[1:batch * rows + 1], want[:batch * rows],
                                    f"{name} B{batch} Q{bits} g{group} {rows}x{cols}")


def test_dense_blocks_keep_guard_values(gpu):
    for rows in (1, 3, 7, 20):
        for cols in (1, 31, 127, 512):
            i = np.arange(rows * cols)
            w16 = (((i * 7) % 41 - 20) / 32.0).astype(np.float16).view(np.uint16)
            x = ((((np.arange(4 * cols) * 13) % 31) - 15) / 16.0).astype(np.float32)
            want = oracle.dense_f16_f64(w16, x, rows, cols, 4)
            wb = gpu.upload_bytes(np.concatenate([np.zeros(2, np.uint16), w16]))
            xb = gpu.upload_f32(np.concatenate([[99.0], x]))
            for batch in range(1, 5):
                yb = gpu.upload_f32(np.full(batch * rows + 2, 12345.0))
                gpu.dispatch("matmul_f16", [wb, xb, yb], [rows, cols, batch], offsets=[4, 4, 4])
                got = gpu.read_f32(yb, batch * rows + 2)
                assert got[0] == 12345.0 and got[batch * rows + 1] == 12345.0
                block_close(got[1:batch * rows + 1], want[:batch * rows], f"dense {rows}x{cols} B{batch}")
                # tests/batch_matrix.rs:149-166: the block copied at an offset, guards kept.
                cb = gpu.upload_f32(np.full(batch * rows + 2, 54321.0))
                gpu.dispatch("copy_f32", [yb, cb], [batch * rows], offsets=[4, 4])
                copied = gpu.read_f32(cb, batch * rows + 2)
                assert copied[0] == 54321.0 and copied[batch * rows + 1] == 54321.0
                assert np.array_equal(copied[1:batch * rows + 1], got[1:batch * rows + 1])


def test_offset_dispatch_rejects_bounds_and_unsafe_aliases(gpu):
    inp = gpu.upload_f32(np.full(1028, 2.0))
    out = gpu.alloc_f32(1028)
    w = gpu.upload_bytes(np.zeros(512 * 4 // 2, np.uint8))
    s = gpu.upload_f32(np.ones(32))
    b = gpu.upload_f32(np.ones(32))
    cmd = gpu.begin()
    # tests/batch_matrix.rs:176-191: copies need disjoint or identical views.
    for offs in ([0], [2, 0], [0, 2**63], [4, 4]):
        with pytest.raises(qmr.QmrError):
            cmd.encode("copy_f32", [inp, out], [1028], 1028, 128, offs)
    with pytest.raises(qmr.QmrError, match="overlaps input buffer 0"):
        cmd.encode("copy_f32", [inp, inp], [32], 32, 128, [0, 4])
    cmd.encode("copy_f32", [inp, inp], [32], 32, 128, [4, 4])
    # Misaligned and out-of-range views are rejected before anything is enqueued.
    for offs in ([0, 0, 0, 2, 0], [0, 0, 0, 0, 2**63], [0, 0, 0, 4, 4100]):
        with pytest.raises(qmr.QmrError):
            cmd.encode("matvec_affine", [w, s, b, inp, out], [4, 512, 4, 64], 128, 128, offs)
    with pytest.raises(qmr.QmrError, match="offset count"):
        cmd.encode("matvec_affine", [w, s, b, inp, out], [4, 512, 4, 64], 128, 128, [0, 0])
    with pytest.raises(qmr.QmrError, match="expected 128 threads"):
        cmd.encode("matvec_affine", [w, s, b, inp, out], [4, 512, 4, 64], 96, 128)
    with pytest.raises(qmr.QmrError, match="threadgroup size"):
        cmd.encode("matvec_affine", [w, s, b, inp, out], [4, 512, 4, 64], 128, 48)
    # Scalar offset matvec KAT: zero codes, s=b=1, x=2 -> 1024.
    cmd.encode("matvec_affine", [w, s, b, inp, out], [4, 512, 4, 64], 128, 128, [0, 0, 0, 4, 4])
    # A BF16 matvec needs a 16-byte aligned input view.
    s16 = gpu.upload_bytes(np.zeros(64, np.uint8))
    with pytest.raises(qmr.QmrError, match="16-byte aligned"):
        cmd.encode("matvec_affine_bf16", [w, s16, s16, inp, out], [4, 512, 4, 64], 128, 128,
                   [0, 0, 0, 4, 4])
    # A block output may not overlap any input view of the same buffer.
    with pytest.raises(qmr.QmrError, match="overlaps input buffer 3"):
        cmd.encode("matmul_affine", [w, s, b, inp, inp], [4, 512, 4, 64, 1], 128, 128,
                   [0, 0, 0, 0, 8])
    cmd.finish()
    cmd.release()
    got = gpu.read_f32(out, 1028)
    assert got[0] == 0.0 and got[5] == 0.0 and got[1027] == 0.0
    assert got[1:5].tolist() == [1024.0] * 4


def _aligned_case(rows, cols):
    i = np.arange(rows * cols // 8, dtype=np.uint64)
    w = ((i * 0x1478ABCF + 0x9E3779B9) & 0xFFFFFFFF).astype(np.uint32)
    k = np.arange(rows * cols // 64)
    s = ((1 + k % 11) * 0.001953125).astype(np.float32)
    b = ((k % 9) * 0.00390625 - 0.0625).astype(np.float32)
    return w, s, b


def test_aligned_q4_blocks_match_oracle_sequential_path_and_every_schedule(gpu):
    legacy = {}
    try:
        for mode in ("legacy", "shared", "mlp-r2"):
            gpu.set_block_kernel_mode(mode, False)
            for cols in (512, 5120, 17408):
                rows = 20
                w, s, b = _aligned_case(rows, cols)
                x = ((((np.arange(4 * cols) * 13) % 101) - 50) / 50).astype(np.float32)
                wb = gpu.upload_bytes(w)
                xb = gpu.upload_f32(x)
                for bf16 in (False, True):
                    sm = (s.view(np.uint32) >> 16).astype(np.uint16) if bf16 else s
                    bm = (b.view(np.uint32) >> 16).astype(np.uint16) if bf16 else b
                    want = oracle.matmul_f64(w, sm, bm, "bf16" if bf16 else "f32", x, rows, cols,
                                             4, 64, 4)
                    sb, bb = gpu.upload_bytes(sm), gpu.upload_bytes(bm)
                    mm = "matmul_affine_bf16" if bf16 else "matmul_affine"
                    mv = "matvec_affine_bf16" if bf16 else "matvec_affine"
                    for batch in range(1, 5):
                        y = gpu.alloc_f32(rows * batch)
                        seq = gpu.alloc_f32(rows * batch)
                        cmd = gpu.begin()
                        cmd.encode(mm, [wb, sb, bb, xb, y], [rows, cols, 4, 64, batch], rows * 32, 128)
                        for t in range(batch):
                            cmd.encode(mv, [wb, sb, bb, xb, seq], [rows, cols, 4, 64], rows * 32,
                                       128, [0, 0, 0, t * cols * 4, t * rows * 4])
                        cmd.finish()
                        cmd.release()
                        got = gpu.read_f32(y, rows * batch)
                        block_close(got, want[:rows * batch], f"{mode} B{batch} cols{cols} bf16={bf16}")
                        key = (cols, bf16, batch)
                        if mode == "legacy":
                            legacy[key] = got.copy()
                        else:
                            assert np.array_equal(got.view(np.uint32), legacy[key].view(np.uint32)), \
                                f"{mode} must preserve every bit B{batch} cols{cols} bf16={bf16}"
                        sq = gpu.read_f32(seq, rows * batch)
                        assert_close_ref(got, sq, 1e-5, 3e-6, f"block vs sequential {key}")
    finally:
        gpu.set_block_kernel_mode("legacy", True)


def test_stream_offset_weights_fall_back_to_packed_alignment(gpus):
    gpu = gpus["stream"]
    vals = np.concatenate([[0], np.full(4 * 512 // 8, 0x76543210)]).astype(np.uint32)
    w = gpu.upload_bytes(vals)
    s = gpu.upload_f32(np.ones(32))
    b = gpu.upload_f32(np.zeros(32))
    x = gpu.upload_f32(np.ones(512))
    y = gpu.alloc_f32(4)
    gpu.dispatch("matvec_affine", [w, s, b, x, y], [4, 512, 4, 64], offsets=[4, 0, 0, 0, 0])
    assert gpu.last_kernel() == "matvec_q4_g64"
    assert gpu.read_f32(y, 4).tolist() == [1792.0] * 4


@pytest.mark.parametrize("rows,cols", [(17408, 5120), (5120, 17408)])
def test_selective_mlp_r2_real_shapes_match_legacy_bits_and_fp64_with_guards(gpu, rows, cols):
    w, s, b = _aligned_case(rows, cols)
    x = ((((np.arange(3 * cols) * 13) % 101) - 50) / 50).astype(np.float32)
    s16 = (s.view(np.uint32) >> 16).astype(np.uint16)
    b16 = (b.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(s16.astype(np.uint32) << 16, s.view(np.uint32)), "exact BF16 fixture"
    guard = lambda a: gpu.upload_bytes(np.concatenate([np.full(16, 0xA5, np.uint8),
                                                       np.frombuffer(a.tobytes(), np.uint8),
                                                       np.full(16, 0xA5, np.uint8)]))
    wb, sb, bb, xb = guard(w), guard(s16), guard(b16), guard(x)
    outs, kernels = [], []
    labels = {"legacy": "matmul_q4_g64_b3_aligned_bf16", "mlp-r2": "matmul_q4_g64_b3_mlp_r2_aligned_bf16",
              "shared": "matmul_q4_g64_b3_shared_aligned_bf16"}
    try:
        for mode in ("legacy", "mlp-r2", "shared"):
            gpu.set_block_kernel_mode(mode, True)
            y = gpu.upload_f32(np.full(rows * 3 + 8, 12345.0))
            gpu.dispatch("matmul_affine_bf16", [wb, sb, bb, xb, y], [rows, cols, 4, 64, 3],
                         offsets=[16] * 5)
            assert gpu.last_kernel() == labels[mode]
            kernels.append(gpu.last_hip_kernel())
            outs.append(gpu.read_f32(y, rows * 3 + 8))
    finally:
        gpu.set_block_kernel_mode("legacy", True)
    # The schedules run their own instances of the row-band kernel with the
    # legacy splits and waves, so every row's sums are the same operations:
    # shared takes the other ring depth; R2 halves (else doubles) the row
    # tiles per band where that shape has a one-round plan, which at
    # 5120x17408 B=3 neither has (its x images leave one workgroup per CU,
    # and eight tiles of two waves exceed 512 threads), so there R2 runs the
    # legacy instance.
    assert all(k.startswith("affine_band_kernel") for k in kernels), kernels
    assert kernels[2] != kernels[0], kernels
    if (rows, cols) == (17408, 5120):
        assert len(set(kernels)) == 3, kernels
    else:
        assert kernels[1] == kernels[0], kernels
    for got in outs:
        assert (got[:4] == 12345.0).all() and (got[rows * 3 + 4:] == 12345.0).all()
        assert np.isfinite(got[4:rows * 3 + 4]).all()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))
    sample = [k * (rows - 1) // 31 for k in range(32)]
    sub = lambda a, per: np.concatenate([a[r * per:(r + 1) * per] for r in sample])
    want = oracle.matmul_f64(sub(w, cols // 8), sub(s16, cols // 64), sub(b16, cols // 64), "bf16",
                             x, len(sample), cols, 4, 64, 3)
    got = np.concatenate([outs[0][4 + t * rows + np.array(sample)] for t in range(3)])
    block_close(got, want, "full MLP sampled rows")
    for buf, arr in ((wb, w), (sb, s16), (bb, b16), (xb, x)):
        raw = np.frombuffer(buf.read_bytes(), np.uint8)
        assert (raw[:16] == 0xA5).all() and (raw[-16:] == 0xA5).all(), "input guard changed"
        assert raw[16:-16].tobytes() == arr.tobytes(), "input changed"

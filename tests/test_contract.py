"""Host-side dispatch contract of libqmr_hip.so, tested on the CPU through the
C ABI. Each test restates one of the reference's host-only tests of the
Metal backend (src/gpu.rs:1295-1634, src/gpu/metadata.rs:20-71) against
this library's routines of the same names.
"""
import numpy as np
import pytest

import qmr

U32_MAX = 0xFFFFFFFF


def err(fn, *a):
    with pytest.raises(qmr.QmrError):
        fn(*a)


# src/gpu.rs:1298-1323
def test_block_kernel_device_defaults_are_limited_to_measured_m5_pro():
    for name, want in [("Apple M5 Pro", "mlp-r2"), ("Apple M5", "legacy"), ("Apple M5 Max", "legacy"),
                       ("Apple M1", "legacy"), ("Apple M1 Pro", "legacy"), ("Apple M4 Pro", "legacy"),
                       ("Apple M5 Pro Max", "legacy"), ("apple m5 pro", "legacy"),
                       ("Apple M5 Pro ", "legacy"), ("", "legacy"),
                       ("AMD Instinct MI355X", "legacy")]:
        assert qmr.parse_block_kernel_mode(name) == (want, True), name


# src/gpu.rs:1325-1352
def test_block_kernel_explicit_modes_override_device_defaults():
    for name in ("Apple M5 Pro", "Apple M1"):
        for matmul in ("legacy", "shared", "mlp-r2"):
            for delta, batched in (("sequential", False), ("batched", True)):
                assert qmr.parse_block_kernel_mode(name, matmul, delta) == (matmul, batched)
    assert qmr.parse_block_kernel_mode("Apple M5 Pro", None, "sequential") == ("mlp-r2", False)


# src/gpu.rs:1354-1367, 1369-1398
def test_block_kernel_modes_reject_unknown_values():
    for name in ("Apple M5 Pro", "Apple M1"):
        for bad in ("", "auto", "LEGACY", "legacy ", "mlp_r2", "MLP-R2", "SHARED", "shared "):
            err(qmr.parse_block_kernel_mode, name, bad, None)
            err(qmr.parse_block_kernel_mode, name, None, bad)


# src/gpu.rs:1400-1430
def test_shared_matmul_selection_changes_only_supported_aligned_batches():
    for batch in range(1, 5):
        for name in ("matmul_affine", "matmul_affine_bf16"):
            p = [20, 5120, 4, 64, batch]
            legacy = qmr.specialized_matmul(name, p, True, "legacy")
            shared = qmr.specialized_matmul(name, p, True, "shared")
            assert "_shared" not in legacy
            assert ("_shared" in shared) == (batch in (2, 3))
            if batch in (1, 4):
                assert legacy == shared
            for fb, aligned in ((p, False), ([19, 5120, 4, 64, batch], True),
                                ([20, 5120, 8, 64, batch], True), ([20, 5120, 4, 32, batch], True)):
                assert qmr.specialized_matmul(name, fb, aligned, "legacy") == \
                    qmr.specialized_matmul(name, fb, aligned, "shared")


# src/gpu.rs:1431-1478
def test_mlp_r2_selection_is_limited_to_measured_shapes_and_format():
    for rows, cols in [(17408, 5120), (5120, 17408), (248320, 5120), (20, 5120), (17408, 512),
                       (17412, 5120)]:
        for batch in range(1, 5):
            for name in ("matmul_affine", "matmul_affine_bf16"):
                for bits, group in ((4, 32), (4, 64), (4, 128), (8, 64)):
                    for aligned in (False, True):
                        p = [rows, cols, bits, group, batch]
                        want_r2 = (aligned and name == "matmul_affine_bf16" and batch == 3 and
                                   bits == 4 and group == 64 and (rows, cols) in
                                   ((17408, 5120), (5120, 17408)))
                        got = qmr.specialized_matmul(name, p, aligned, "mlp-r2")
                        if want_r2:
                            assert got == "matmul_q4_g64_b3_mlp_r2_aligned_bf16"
                        else:
                            assert got == qmr.specialized_matmul(name, p, aligned, "legacy")
            dense = [rows, cols, batch]
            assert qmr.specialized_matmul("matmul_f16", dense, True, "mlp-r2") == \
                qmr.specialized_matmul("matmul_f16", dense, True, "legacy")


# src/gpu.rs:1479-1488
def test_buffer_views_reject_misalignment_bounds_and_integer_wraparound():
    qmr.checked_buffer_range(4, 12, 16)
    qmr.checked_buffer_range(0, 16, 16)
    err(qmr.checked_buffer_range, 4, 16, 16)
    err(qmr.checked_buffer_range, 2, 12, 16)
    err(qmr.checked_buffer_range, 2**64 - 4, 8, 2**64 - 1)
    assert qmr.ranges_overlap(0, 8, 4, 8)
    assert not qmr.ranges_overlap(0, 8, 8, 8)


# src/gpu.rs:1489-1536
def test_block_specialization_preserves_alignment_and_all_batch_sizes():
    for batch in range(1, 5):
        p = [20, 5120, 4, 64, batch]
        assert qmr.specialized_matmul("matmul_affine", p, True).endswith("_aligned")
        assert qmr.specialized_matmul("matmul_affine_bf16", p, True).endswith("_aligned_bf16")
        assert not qmr.specialized_matmul("matmul_affine", p, False).endswith("_aligned")
        assert not qmr.specialized_matmul("matmul_affine", [19, 5120, 4, 64, batch], True).endswith("_aligned")
        assert not qmr.specialized_matmul("matmul_affine", [20, 5120, 8, 64, batch], True).endswith("_aligned")


# src/gpu.rs:1537-1566
def test_batch_dispatch_layout_sizes_all_rhs_and_rejects_invalid_batches():
    for batch in range(1, 5):
        sizes, threads = qmr.dispatch_layout("matmul_affine", [3, 128, 4, 64, batch])
        assert sizes == [192, 24, 24, 512 * batch, 12 * batch] and threads == 96
        sizes, _ = qmr.dispatch_layout("matmul_affine_bf16", [3, 128, 8, 32, batch])
        assert sizes == [384, 24, 24, 512 * batch, 12 * batch]
        sizes, _ = qmr.dispatch_layout("matmul_f16", [3, 127, batch])
        assert sizes == [762, 508 * batch, 12 * batch]
    for batch in (0, 5, U32_MAX):
        err(qmr.dispatch_layout, "matmul_affine", [3, 128, 4, 64, batch])
        err(qmr.dispatch_layout, "matmul_f16", [3, 127, batch])
    for p in ([3, 127, 4, 64, 2], [3, 256, 4, 256, 2], [3, 128, 2, 64, 2], [U32_MAX, 128, 4, 64, 4]):
        err(qmr.dispatch_layout, "matmul_affine", p)
    err(qmr.dispatch_layout, "matmul_f16", [1, U32_MAX, 4])
    assert qmr.dispatch_layout("copy_f32", [7]) == ([28, 28], 7)
    err(qmr.dispatch_layout, "copy_f32", [0])
    # The read-floor name (a library addition): three byte views, one thread
    # per 16 bytes, 4096 u32 checksum slots.
    assert qmr.dispatch_layout("read_checksum", [44, 8, 0]) == ([44, 8, 0, 16384], 4)
    assert qmr.dispatch_layout("read_checksum", [16, 16, 16]) == ([16, 16, 16, 16384], 3)
    err(qmr.dispatch_layout, "read_checksum", [0, 0, 0])
    err(qmr.dispatch_layout, "read_checksum", [6, 0, 0])
    err(qmr.dispatch_layout, "read_checksum", [16, 16])


# src/gpu.rs:1568-1582
def test_bf16_dispatch_keeps_metadata_typed_and_rejects_unsupported_groups():
    assert qmr.dispatch_layout("matvec_affine_bf16", [20, 5120, 4, 64]) == \
        ([51200, 3200, 3200, 20480, 80], 640)
    assert qmr.dispatch_layout("embed_affine_bf16", [249999, 5120, 4, 64]) == \
        ([640_000_000, 40_000_000, 40_000_000, 20480], 5120)
    for name in ("matvec_affine_bf16", "embed_affine_bf16", "matvec_affine_f16meta",
                 "embed_affine_f16meta"):
        for p in ([2, 256, 4, 256], [2, 128, 4, 8], [2, 128, 2, 64], [2, 127, 4, 64]):
            err(qmr.dispatch_layout, name, p)


# src/gpu.rs:1584-1615
def test_bf16_aligned_kernel_requires_q4_group64_and_safe_dimensions():
    assert qmr.specialized_matvec([20, 5120, 4, 64], True, True) == "matvec_q4_g64_aligned_bf16"
    for p in ([19, 5120, 4, 64], [20, 192, 4, 64], [524288, 8192, 4, 64]):
        assert qmr.specialized_matvec(p, True, True) == "matvec_q4_g64_bf16"
    for aligned in (True, False):
        assert qmr.specialized_matvec([20, 5120, 4, 32], aligned, True) == "matvec_q4_g32_bf16"
        assert qmr.specialized_matvec([20, 5120, 4, 128], aligned, True) == "matvec_q4_g128_bf16"
        assert qmr.specialized_matvec([20, 5120, 8, 64], aligned, True) == "matvec_q8_g64_bf16"
        assert qmr.specialized_matvec([20, 5120, 4, 256], aligned, True) is None
    assert qmr.specialized_matvec([20, 5120, 4, 64], False, True) == "matvec_q4_g64_bf16"


# src/gpu.rs:1617-1634
def test_aligned_dispatch_requires_safe_dimensions():
    assert qmr.specialized_matvec([20, 5120, 4, 64], True) == "matvec_q4_g64_aligned"
    for p in ([19, 5120, 4, 64], [20, 192, 4, 64], [524288, 8192, 4, 64]):
        assert qmr.specialized_matvec(p, True) == "matvec_q4_g64"
    assert qmr.specialized_matvec([20, 5120, 4, 256], True) is None
    assert qmr.specialized_matvec([20, 5120, 8, 64], True) == "matvec_q8_g64"
    assert qmr.specialized_matvec([20, 5120, 4, 64], False) == "matvec_q4_g64"


# src/gpu.rs:1677-1688 (matrix part)
def test_rejects_invalid_shapes_and_index_overflow_before_dispatch():
    err(qmr.dispatch_layout, "matvec_affine", [2, 7, 4, 8])
    err(qmr.dispatch_layout, "matvec_affine", [2, 8, 3, 8])
    err(qmr.dispatch_layout, "matvec_f16", [U32_MAX, 2])
    err(qmr.dispatch_layout, "typo", [2])
    err(qmr.dispatch_layout, "matvec_affine", [2, 8, 4])  # parameter count
    err(qmr.dispatch_layout, "matvec_affine", [0, 8, 4, 8])  # nonzero rows
    err(qmr.dispatch_layout, "embed_affine", [0, 0, 4, 8])  # nonzero cols
    with pytest.raises(qmr.QmrError, match="Unknown GPU kernel typo"):
        qmr.dispatch_layout("typo", [2])


# src/gpu.rs:1689-1697
def test_packed_large_vocabulary_uses_checked_sizes():
    assert qmr.dispatch_layout("embed_affine", [249999, 5120, 4, 64]) == \
        ([640_000_000, 80_000_000, 80_000_000, 20480], 5120)


def test_small_group_and_dense_layouts():
    # The KAT shapes of src/gpu.rs:1637-1732 go through the generic layout.
    assert qmr.dispatch_layout("matvec_affine", [2, 8, 4, 8]) == ([8, 8, 8, 32, 8], 64)
    assert qmr.dispatch_layout("matvec_affine", [2, 4, 8, 4]) == ([8, 8, 8, 16, 8], 64)
    assert qmr.dispatch_layout("embed_affine", [0, 4, 8, 4]) == ([4, 4, 4, 16], 4)
    assert qmr.dispatch_layout("matvec_f16", [2, 4]) == ([16, 16, 8], 64)
    assert qmr.dispatch_layout("embed_f16", [1, 4]) == ([16, 16], 4)


def test_added_names_layouts():
    # F16-metadata names: 2-byte metadata like the BF16 names.
    assert qmr.dispatch_layout("matvec_affine_f16meta", [20, 5120, 8, 64]) == \
        ([102400, 3200, 3200, 20480, 80], 640)
    assert qmr.dispatch_layout("matmul_affine_f16meta", [3, 128, 4, 64, 2]) == \
        ([192, 12, 12, 1024, 24], 96)
    # Wide blocks accept 1..256 RHS.
    sizes, threads = qmr.dispatch_layout("matmul_affine_wide_bf16", [17408, 5120, 4, 64, 256])
    assert sizes == [44564480, 2785280, 2785280, 4 * 256 * 5120, 4 * 256 * 17408]
    assert threads == 17408 * 32
    for batch in (0, 257):
        err(qmr.dispatch_layout, "matmul_affine_wide", [16, 512, 4, 64, batch])


def test_fused_names_layouts():
    """The fused forms (no reference counterpart): the residual product takes
    the block's buffers plus r [batch][rows] before y; the MLP form takes the
    gate and up matrices, x, the RMS-norm weights and y, with a finite
    positive epsilon as its sixth word."""
    assert qmr.dispatch_layout("matmul_affine_add_bf16", [3, 128, 4, 64, 2]) == \
        ([192, 12, 12, 1024, 24, 24], 96)
    assert qmr.dispatch_layout("matmul_affine_add", [5120, 17408, 4, 64, 1]) == \
        ([44564480, 5570560, 5570560, 4 * 17408, 4 * 5120, 4 * 5120], 5120 * 32)
    eps = int(np.float32(1e-6).view(np.uint32))
    sizes, threads = qmr.dispatch_layout("mlp_gate_up_swiglu_bf16", [17408, 5120, 4, 64, 3, eps])
    w, m = 17408 * 5120 // 2, 17408 * 80 * 2
    assert sizes == [w, m, m, w, m, m, 4 * 3 * 5120, 4 * 5120, 4 * 3 * 17408] and threads == 17408 * 32
    assert qmr.dispatch_layout("mlp_gate_up_swiglu", [16, 256, 8, 32, 1, eps])[0][1] == 16 * 8 * 4
    for bad in (0, int(np.float32(-1e-6).view(np.uint32)), 0x7F800000, 0x7FC00000):
        with pytest.raises(qmr.QmrError, match="epsilon must be finite and positive"):
            qmr.dispatch_layout("mlp_gate_up_swiglu_f16meta", [16, 256, 4, 64, 1, bad])
    for batch in (0, 5):
        err(qmr.dispatch_layout, "mlp_gate_up_swiglu_bf16", [16, 256, 4, 64, batch, eps])
        err(qmr.dispatch_layout, "matmul_affine_add_bf16", [16, 256, 4, 64, batch])
    err(qmr.dispatch_layout, "mlp_gate_up_swiglu_bf16", [16, 256, 4, 48, 1, eps])
    err(qmr.dispatch_layout, "mlp_gate_up_swiglu_bf16", [16, 256, 4, 64, 1])


# src/gpu/metadata.rs:24-71 through the library's own routine.
def test_pack_bf16_exact_patterns_and_supported_formats():
    patterns = np.array([0x00000000, 0x80000000, 0x3FC00000, 0xC0200000, 0x00010000, 0x80010000,
                         0x00800000, 0x7F7F0000], np.uint32)
    packed = qmr.pack_bf16_exact(patterns.view(np.float32))
    assert ((packed.astype(np.uint32) << 16) == patterns).all()
    for bad in (0.1, np.uint32(1).view(np.float32), np.inf, -np.inf, np.nan):
        assert qmr.pack_bf16_exact(np.array([1.0, bad, -0.0], np.float32)) is None
    for bits in (4, 8):
        for group in (32, 64, 128):
            assert qmr.supported_bf16_quantization(bits, group)
    for bits, group in ((2, 64), (16, 64), (4, 8), (4, 256), (8, 0)):
        assert not qmr.supported_bf16_quantization(bits, group)


@pytest.mark.parametrize("rows,cols,batch", [(17408, 5120, 128), (17408, 5120, 256), (5120, 17408, 64),
                                             (16 * 17 * 3 + 5, 512, 33), (9, 256, 1), (300, 1024, 200)])
@pytest.mark.parametrize("row_tiles", [8, 17])
def test_wide_kernel_loads_stay_inside_their_views(rows, cols, batch, row_tiles):
    """Every code, x-fragment and group-sum load of the wide contraction
    kernel (walked on the host through the kernel's own offset functions):
    loads outside a view go through the vector offset past every view, and
    the in-range ones end inside theirs. The last code byte and the last
    image byte are reached, so the walk covers the views to their ends."""
    code_end, code_extent, image_end, image_extent = qmr.wide_address_extent(rows, cols, batch, row_tiles)
    assert code_end == code_extent == rows * cols // 2
    assert image_extent == (cols // 64) * ((batch + 31) // 32) * 8448
    assert image_end <= image_extent and image_end > image_extent - 8448

"""Python binding of libqmr_hip.so (include/qmr.h) through ctypes.

It mirrors the reference engine's Metal backend interface (`Gpu`,
`DispatchEncoder`, src/gpu.rs:95-876) so that tests and benchmarks read like
the reference's own: a `Gpu` uploads buffers, `begin()` opens a command,
`encode(...)` checks and enqueues one dispatch by reference kernel name and
`finish()` synchronises and returns the frame timing.

The library is built by qwen-mlx-runner_amd/build.py. Loading fails loudly if
it is missing: there is no CPU fallback behind this interface.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_DIR / "libqmr_hip.so"

QMR_OK = 0
QMR_ERR_INVALID = 1
QMR_ERR_DEVICE = 2
QMR_ERR_UNSUPPORTED = 3

BLOCK_MODES = {"legacy": 0, "shared": 1, "mlp-r2": 2}
BLOCK_MODE_NAMES = {v: k for k, v in BLOCK_MODES.items()}
# Output slots of the read_checksum kernel (u32; their XOR is the XOR of every
# word read).
CHECKSUM_SLOTS = 4096
# Bytes of the static scratch behind qmr_encode_static (QMR_STATIC_SCRATCH_BYTES).
STATIC_SCRATCH_BYTES = 8 << 20

EXPORTED_SYMBOLS = (
    "qmr_last_error", "qmr_device_open", "qmr_device_close", "qmr_device_name",
    "qmr_kernel_mode", "qmr_metadata_mode", "qmr_block_kernel_mode",
    "qmr_set_block_kernel_mode", "qmr_compact_metadata", "qmr_record_compacted_metadata",
    "qmr_metadata_stats", "qmr_buffer_alloc", "qmr_buffer_upload", "qmr_buffer_read",
    "qmr_buffer_write", "qmr_buffer_length", "qmr_buffer_retain", "qmr_buffer_release",
    "qmr_command_begin", "qmr_encode", "qmr_encode_static", "qmr_command_mark", "qmr_command_delay",
    "qmr_command_finish",
    "qmr_command_elapsed", "qmr_command_release", "qmr_dispatch_layout",
    "qmr_checked_buffer_range", "qmr_ranges_overlap", "qmr_specialized_matvec",
    "qmr_specialized_matmul", "qmr_parse_block_kernel_mode", "qmr_pack_bf16_exact",
    "qmr_supported_bf16_quantization", "qmr_set_gemv_plan", "qmr_gemv_plan", "qmr_wide_address_extent",
    "qmr_last_kernel", "qmr_last_hip_kernel", "qmr_device_max_lds", "qmr_set_band_wait_fault",
    "qmr_device_workspace_bytes", "qmr_set_read_plan",
    # include/qmr_checkpoint.h
    "qmr_checkpoint_open", "qmr_checkpoint_close", "qmr_checkpoint_tensor_count",
    "qmr_checkpoint_contains", "qmr_checkpoint_matrix_info", "qmr_checkpoint_matrix",
    "qmr_checkpoint_dense", "qmr_matrix_load", "qmr_matrix_release",
)


class QmrError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class _Options(C.Structure):
    _fields_ = [("gemv_variant", C.c_char_p), ("metadata_mode", C.c_char_p),
                ("block_matmul", C.c_char_p), ("block_delta", C.c_char_p),
                ("reference", C.c_int)]


class _Timing(C.Structure):
    _fields_ = [("cpu_encode_seconds", C.c_double), ("cpu_commit_seconds", C.c_double),
                ("gpu_seconds", C.c_double), ("completion_wait_seconds", C.c_double)]


class _MatrixInfo(C.Structure):
    _fields_ = [("packed", C.c_int), ("rows", C.c_size_t), ("cols", C.c_size_t),
                ("bits", C.c_uint32), ("group_size", C.c_size_t), ("dtype", C.c_char * 8),
                ("metadata_dtype", C.c_char * 8)]


class _Matrix(C.Structure):
    _fields_ = [("weight", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("rows", C.c_size_t), ("cols", C.c_size_t), ("bits", C.c_uint32),
                ("group", C.c_size_t), ("metadata_bf16", C.c_int)]


@dataclass
class FrameTiming:
    """FrameTiming of src/gpu/timing.rs:8-21."""
    cpu_encode_seconds: float
    cpu_commit_seconds: float
    gpu_seconds: float
    completion_wait_seconds: float


_lib: Optional[C.CDLL] = None
_alive = True  # cleared at interpreter exit: no handle is released after that


def _at_exit() -> None:
    global _alive
    _alive = False


atexit.register(_at_exit)


def lib() -> C.CDLL:
    """Load libqmr_hip.so once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("QMR_LIB", LIB_PATH))
    if not path.exists():
        raise ImportError(f"{path} is missing: build it with python qwen-mlx-runner_amd/build.py")
    L = C.CDLL(str(path))
    vp, sz, u32p, szp = C.c_void_p, C.c_size_t, C.POINTER(C.c_uint32), C.POINTER(C.c_size_t)
    sig = {
        "qmr_last_error": (C.c_char_p, []),
        "qmr_device_open": (C.c_int, [C.c_int, C.POINTER(_Options), C.POINTER(vp)]),
        "qmr_device_close": (None, [vp]),
        "qmr_device_name": (C.c_char_p, [vp]),
        "qmr_kernel_mode": (C.c_char_p, [vp]),
        "qmr_metadata_mode": (C.c_char_p, [vp]),
        "qmr_block_kernel_mode": (None, [vp, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "qmr_set_block_kernel_mode": (C.c_int, [vp, C.c_int, C.c_int]),
        "qmr_compact_metadata": (C.c_int, [vp, C.c_uint32, sz, vp, vp, sz, vp, vp]),
        "qmr_record_compacted_metadata": (None, [vp, C.c_uint64]),
        "qmr_metadata_stats": (None, [vp, szp, C.POINTER(C.c_uint64)]),
        "qmr_buffer_alloc": (C.c_int, [vp, sz, C.POINTER(vp)]),
        "qmr_buffer_upload": (C.c_int, [vp, vp, sz, C.POINTER(vp)]),
        "qmr_buffer_read": (C.c_int, [vp, sz, vp, sz]),
        "qmr_buffer_write": (C.c_int, [vp, sz, vp, sz]),
        "qmr_buffer_length": (sz, [vp]),
        "qmr_buffer_retain": (None, [vp]),
        "qmr_buffer_release": (None, [vp]),
        "qmr_command_begin": (C.c_int, [vp, C.POINTER(vp)]),
        "qmr_encode": (C.c_int, [vp, C.c_char_p, C.POINTER(vp), szp, sz, u32p, sz, sz, sz]),
        "qmr_wide_address_extent": (C.c_int, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint64)]),
        "qmr_encode_static": (C.c_int, [vp, C.c_char_p, C.POINTER(vp), szp, sz, u32p, sz, sz, sz]),
        "qmr_command_mark": (C.c_int, [vp, C.POINTER(C.c_int)]),
        "qmr_command_delay": (C.c_int, [vp, C.c_uint32]),
        "qmr_command_finish": (C.c_int, [vp, C.POINTER(_Timing)]),
        "qmr_command_elapsed": (C.c_int, [vp, C.c_int, C.c_int, C.POINTER(C.c_double)]),
        "qmr_command_release": (None, [vp]),
        "qmr_dispatch_layout": (C.c_int, [C.c_char_p, u32p, sz, szp, sz, szp, szp]),
        "qmr_checked_buffer_range": (C.c_int, [sz, sz, sz]),
        "qmr_ranges_overlap": (C.c_int, [sz, sz, sz, sz]),
        "qmr_specialized_matvec": (C.c_char_p, [u32p, C.c_int, C.c_int]),
        "qmr_specialized_matmul": (C.c_char_p, [C.c_char_p, u32p, sz, C.c_int, C.c_int]),
        "qmr_parse_block_kernel_mode": (C.c_int, [C.c_char_p, C.c_char_p, C.c_char_p,
                                                  C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "qmr_pack_bf16_exact": (C.c_int, [vp, sz, vp]),
        "qmr_supported_bf16_quantization": (C.c_int, [C.c_uint32, sz]),
        "qmr_set_gemv_plan": (C.c_int, [vp, C.c_int, C.c_int]),
        "qmr_gemv_plan": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                    C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "qmr_last_kernel": (C.c_char_p, [vp]),
        "qmr_last_hip_kernel": (C.c_char_p, [vp]),
        "qmr_device_max_lds": (sz, [vp]),
        "qmr_set_band_wait_fault": (C.c_int, [vp, C.c_int]),
        "qmr_device_workspace_bytes": (sz, [vp]),
        "qmr_set_read_plan": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_int]),
        "qmr_checkpoint_open": (C.c_int, [C.c_char_p, C.POINTER(vp)]),
        "qmr_checkpoint_close": (None, [vp]),
        "qmr_checkpoint_tensor_count": (sz, [vp]),
        "qmr_checkpoint_contains": (C.c_int, [vp, C.c_char_p]),
        "qmr_checkpoint_matrix_info": (C.c_int, [vp, C.c_char_p, C.POINTER(_MatrixInfo)]),
        "qmr_checkpoint_matrix": (C.c_int, [vp, C.c_char_p, vp, vp, vp]),
        "qmr_checkpoint_dense": (C.c_int, [vp, C.c_char_p, vp]),
        "qmr_matrix_load": (C.c_int, [vp, vp, C.c_char_p, sz, sz, C.POINTER(_Matrix)]),
        "qmr_matrix_release": (None, [C.POINTER(_Matrix)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(code: int) -> None:
    if code != QMR_OK:
        raise QmrError(code, lib().qmr_last_error().decode())


def _u32(params: Sequence[int]):
    arr = (C.c_uint32 * max(len(params), 1))(*[int(p) & 0xFFFFFFFF for p in params])
    return arr


def _s(v: Optional[str]) -> Optional[bytes]:
    return None if v is None else v.encode()


# ---- host-only contract (no GPU needed) ----

def wide_address_extent(rows: int, cols: int, batch: int, row_tiles: int) -> tuple[int, int, int, int]:
    """qmr_wide_address_extent: (largest end of the wide kernel's in-range code
    loads, code view bytes, largest end of its in-range image loads, image
    workspace bytes), walked on the host."""
    out = (C.c_uint64 * 4)()
    _check(lib().qmr_wide_address_extent(rows, cols, batch, row_tiles, out))
    return tuple(int(v) for v in out)


def dispatch_layout(name: str, params: Sequence[int]) -> tuple[list[int], int]:
    """dispatch_layout (src/gpu.rs:1041-1294) for the matrix kernels."""
    sizes = (C.c_size_t * 16)()
    n = C.c_size_t()
    threads = C.c_size_t()
    _check(lib().qmr_dispatch_layout(name.encode(), _u32(params), len(params), sizes, 16,
                                     C.byref(n), C.byref(threads)))
    return [sizes[i] for i in range(n.value)], threads.value


def checked_buffer_range(offset: int, minimum: int, length: int) -> None:
    _check(lib().qmr_checked_buffer_range(offset, minimum, length))


def ranges_overlap(a: int, a_len: int, b: int, b_len: int) -> bool:
    return bool(lib().qmr_ranges_overlap(a, a_len, b, b_len))


def specialized_matvec(params: Sequence[int], aligned: bool, bf16: bool = False) -> Optional[str]:
    r = lib().qmr_specialized_matvec(_u32(params), int(aligned), int(bf16))
    return None if r is None else r.decode()


def specialized_matmul(name: str, params: Sequence[int], aligned: bool,
                       mode: str = "legacy") -> Optional[str]:
    r = lib().qmr_specialized_matmul(name.encode(), _u32(params), len(params), int(aligned),
                                     BLOCK_MODES[mode])
    return None if r is None else r.decode()


def parse_block_kernel_mode(device_name: str, matmul: Optional[str] = None,
                            delta: Optional[str] = None) -> tuple[str, bool]:
    m, d = C.c_int(), C.c_int()
    _check(lib().qmr_parse_block_kernel_mode(device_name.encode(), _s(matmul), _s(delta),
                                             C.byref(m), C.byref(d)))
    return BLOCK_MODE_NAMES[m.value], bool(d.value)


def pack_bf16_exact(values: np.ndarray) -> Optional[np.ndarray]:
    v = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(v.size, dtype=np.uint16)
    ok = lib().qmr_pack_bf16_exact(v.ctypes.data, v.size, out.ctypes.data)
    return out if ok else None


def supported_bf16_quantization(bits: int, group: int) -> bool:
    return bool(lib().qmr_supported_bf16_quantization(bits, group))


# ---- device objects ----

class Buffer:
    """A refcounted device buffer (a Metal buffer handle in the reference)."""

    def __init__(self, handle: int):
        self._h = C.c_void_p(handle)

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def __len__(self) -> int:
        return int(lib().qmr_buffer_length(self._h))

    def read(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        _check(lib().qmr_buffer_read(self._h, offset, out.ctypes.data, out.nbytes))
        return out

    def read_bytes(self, offset: int = 0, nbytes: Optional[int] = None) -> bytes:
        n = len(self) - offset if nbytes is None else nbytes
        out = np.empty(n, dtype=np.uint8)
        _check(lib().qmr_buffer_read(self._h, offset, out.ctypes.data, n))
        return out.tobytes()

    def write(self, data: np.ndarray, offset: int = 0) -> None:
        d = np.ascontiguousarray(data)
        _check(lib().qmr_buffer_write(self._h, offset, d.ctypes.data, d.nbytes))

    def release(self) -> None:
        if self._h:
            lib().qmr_buffer_release(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        if _alive:
            try:
                self.release()
            except Exception:
                pass


class Command:
    """One command: dispatches enqueued on the device stream, then finish()."""

    def __init__(self, gpu: "Gpu", handle: int):
        self.gpu = gpu
        self._h = C.c_void_p(handle)
        self.timing: Optional[FrameTiming] = None

    def encode(self, name: str, buffers: Sequence[Buffer], params: Sequence[int],
               threads: int, group_size: int, offsets: Optional[Sequence[int]] = None,
               static_scratch: bool = False) -> None:
        """DispatchEncoder::encode / encode_offsets (src/gpu.rs:120-141).
        static_scratch=True calls qmr_encode_static instead: the same launch
        with its workspace in the GPU's static scratch, allocating nothing."""
        n = len(buffers)
        bufs = (C.c_void_p * max(n, 1))(*[b.handle.value for b in buffers])
        offs = None
        if offsets is not None:
            if len(offsets) != n:
                raise QmrError(QMR_ERR_INVALID, f"{name}: offset count must match buffers")
            offs = (C.c_size_t * max(n, 1))(*[int(o) for o in offsets])
        entry = lib().qmr_encode_static if static_scratch else lib().qmr_encode
        _check(entry(self._h, name.encode(), bufs, offs, n, _u32(params), len(params), threads, group_size))

    def mark(self) -> int:
        idx = C.c_int()
        _check(lib().qmr_command_mark(self._h, C.byref(idx)))
        return idx.value

    def delay(self, microseconds: int) -> None:
        """Hold the device stream for `microseconds` of GPU time (at most
        1,000,000), so that launches encoded next are queued before the GPU
        reaches them (a measurement aid; no reference counterpart)."""
        _check(lib().qmr_command_delay(self._h, int(microseconds)))

    def finish(self) -> FrameTiming:
        t = _Timing()
        _check(lib().qmr_command_finish(self._h, C.byref(t)))
        self.timing = FrameTiming(t.cpu_encode_seconds, t.cpu_commit_seconds, t.gpu_seconds,
                                  t.completion_wait_seconds)
        return self.timing

    def elapsed_ms(self, a: int, b: int) -> float:
        v = C.c_double()
        _check(lib().qmr_command_elapsed(self._h, a, b, C.byref(v)))
        return v.value

    def release(self) -> None:
        if self._h:
            lib().qmr_command_release(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        if _alive:
            try:
                self.release()
            except Exception:
                pass


class Gpu:
    """Gpu::new_with_variant (src/gpu.rs:305-437) on a HIP device."""

    def __init__(self, variant: str = "aligned", reference: bool = False,
                 metadata: str = "f32", block_matmul: Optional[str] = None,
                 block_delta: Optional[str] = None, ordinal: int = 0):
        opts = _Options(_s(variant), _s(metadata), _s(block_matmul), _s(block_delta),
                        int(reference))
        h = C.c_void_p()
        _check(lib().qmr_device_open(ordinal, C.byref(opts), C.byref(h)))
        self._h = h

    # -- properties
    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def name(self) -> str:
        return lib().qmr_device_name(self._h).decode()

    def kernel_mode(self) -> str:
        return lib().qmr_kernel_mode(self._h).decode()

    def metadata_mode(self) -> str:
        return lib().qmr_metadata_mode(self._h).decode()

    def block_kernel_mode(self) -> tuple[str, bool]:
        m, d = C.c_int(), C.c_int()
        lib().qmr_block_kernel_mode(self._h, C.byref(m), C.byref(d))
        return BLOCK_MODE_NAMES[m.value], bool(d.value)

    def set_block_kernel_mode(self, matmul: str, batched_delta: bool = True) -> None:
        _check(lib().qmr_set_block_kernel_mode(self._h, BLOCK_MODES[matmul], int(batched_delta)))

    def set_gemv_plan(self, rr: int = 0, ks: int = 0) -> None:
        _check(lib().qmr_set_gemv_plan(self._h, rr, ks))

    def set_band_wait_fault(self, enabled: bool) -> None:
        """Testing hook: the row-band and split-K kernels' last splits give
        up (their command's finish then fails)."""
        _check(lib().qmr_set_band_wait_fault(self._h, int(enabled)))

    def set_read_plan(self, workgroups: int = 0, unroll: int = 0, nontemporal: int = -1) -> None:
        """read_checksum's geometry (zeros and -1: the defaults)."""
        _check(lib().qmr_set_read_plan(self._h, workgroups, unroll, nontemporal))

    def workspace_bytes(self) -> int:
        """Device workspace this handle has allocated (split sums, split-K
        partials and counters, wide-block images)."""
        return int(lib().qmr_device_workspace_bytes(self._h))

    def gemv_plan(self, rows: int, cols: int, bits: int, batch: int) -> tuple[int, int]:
        rr, ks = C.c_int(), C.c_int()
        _check(lib().qmr_gemv_plan(self._h, rows, cols, bits, batch, C.byref(rr), C.byref(ks)))
        return rr.value, ks.value

    def last_kernel(self) -> str:
        return lib().qmr_last_kernel(self._h).decode()

    def last_hip_kernel(self) -> str:
        """The HIP kernel (and row-band plan) the last encode launched."""
        return lib().qmr_last_hip_kernel(self._h).decode()

    def max_lds(self) -> int:
        return int(lib().qmr_device_max_lds(self._h))

    def compact_metadata(self, bits: int, group: int, scales: np.ndarray, biases: np.ndarray):
        s = np.ascontiguousarray(scales, dtype=np.float32)
        b = np.ascontiguousarray(biases, dtype=np.float32)
        so = np.empty(s.size, np.uint16)
        bo = np.empty(b.size, np.uint16)
        ok = lib().qmr_compact_metadata(self._h, bits, group, s.ctypes.data, b.ctypes.data,
                                        s.size, so.ctypes.data, bo.ctypes.data)
        return (so, bo) if ok else None

    def metadata_stats(self) -> tuple[int, int]:
        """Gpu::metadata_stats (src/gpu.rs:491-496): matrices whose metadata was
        compacted to BF16, and the bytes that saved."""
        n, saved = C.c_size_t(), C.c_uint64()
        lib().qmr_metadata_stats(self._h, C.byref(n), C.byref(saved))
        return n.value, saved.value

    # -- buffers (src/gpu.rs:540-589)
    def alloc(self, nbytes: int) -> Buffer:
        h = C.c_void_p()
        _check(lib().qmr_buffer_alloc(self._h, nbytes, C.byref(h)))
        return Buffer(h.value)

    def alloc_f32(self, n: int) -> Buffer:
        return self.alloc(4 * n)

    def upload_bytes(self, data) -> Buffer:
        arr = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray))
                                   else data)
        h = C.c_void_p()
        _check(lib().qmr_buffer_upload(self._h, arr.ctypes.data if arr.nbytes else None,
                                       arr.nbytes, C.byref(h)))
        return Buffer(h.value)

    def upload_f32(self, values) -> Buffer:
        return self.upload_bytes(np.ascontiguousarray(values, dtype=np.float32))

    def read_f32(self, buf: Buffer, n: int, offset: int = 0) -> np.ndarray:
        return buf.read(np.float32, n, offset)

    # -- commands (src/gpu.rs:590-876)
    def begin(self) -> Command:
        h = C.c_void_p()
        _check(lib().qmr_command_begin(self._h, C.byref(h)))
        return Command(self, h.value)

    def dispatch(self, name: str, buffers: Sequence[Buffer], params: Sequence[int],
                 offsets: Optional[Sequence[int]] = None, group_size: int = 128) -> FrameTiming:
        """One dispatch in its own command, with the layout's thread count."""
        _, threads = dispatch_layout(name, params)
        cmd = self.begin()
        try:
            cmd.encode(name, buffers, params, threads, group_size, offsets)
            return cmd.finish()
        finally:
            cmd.release()

    def close(self) -> None:
        if self._h:
            lib().qmr_device_close(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        if _alive:
            try:
                self.close()
            except Exception:
                pass


# ---- checkpoints (include/qmr_checkpoint.h) ----

@dataclass
class MatrixInfo:
    """What Checkpoint::matrix (src/weights.rs:292-351) returns, without the data."""
    packed: bool
    rows: int
    cols: int
    bits: int
    group_size: int
    dtype: str
    metadata_dtype: str


@dataclass
class PackedData:
    """MatrixData::Packed (src/weights.rs:15-29): words and FP32 metadata."""
    rows: int
    cols: int
    bits: int
    group_size: int
    weights: np.ndarray
    scales: np.ndarray
    biases: np.ndarray


@dataclass
class DenseData:
    """MatrixData::Dense: F16 bit patterns, row-major."""
    rows: int
    cols: int
    values: np.ndarray


@dataclass
class Matrix:
    """A matrix resident on one device (`Matrix`, src/engine.rs:22-31)."""
    weight: Buffer
    scales: Optional[Buffer]
    biases: Optional[Buffer]
    rows: int
    cols: int
    bits: int
    group: int
    metadata_bf16: bool


class Checkpoint:
    """Checkpoint (src/weights.rs:47-486): an MLX safetensors checkpoint,
    memory-mapped and validated when opened."""

    def __init__(self, path: str | os.PathLike):
        h = C.c_void_p()
        _check(lib().qmr_checkpoint_open(os.fsencode(os.fspath(path)), C.byref(h)))
        self._h = h

    def __len__(self) -> int:
        return int(lib().qmr_checkpoint_tensor_count(self._h))

    def contains(self, name: str) -> bool:
        return bool(lib().qmr_checkpoint_contains(self._h, name.encode()))

    def matrix_info(self, name: str) -> MatrixInfo:
        i = _MatrixInfo()
        _check(lib().qmr_checkpoint_matrix_info(self._h, name.encode(), C.byref(i)))
        return MatrixInfo(bool(i.packed), i.rows, i.cols, i.bits, i.group_size,
                          i.dtype.decode(), i.metadata_dtype.decode())

    def matrix(self, name: str) -> PackedData | DenseData:
        i = self.matrix_info(name)
        if not i.packed:
            v = np.empty(i.rows * i.cols, np.uint16)
            _check(lib().qmr_checkpoint_dense(self._h, name.encode(), v.ctypes.data))
            return DenseData(i.rows, i.cols, v)
        w = np.empty(i.rows * i.cols // (32 // i.bits), np.uint32)
        g = i.rows * i.cols // i.group_size
        sc, bi = np.empty(g, np.float32), np.empty(g, np.float32)
        _check(lib().qmr_checkpoint_matrix(self._h, name.encode(), w.ctypes.data, sc.ctypes.data,
                                           bi.ctypes.data))
        return PackedData(i.rows, i.cols, i.bits, i.group_size, w, sc, bi)

    def load(self, gpu: "Gpu", name: str, rows: int, cols: int) -> Matrix:
        """Matrix::load (src/engine.rs:48-135) into `gpu`'s memory."""
        m = _Matrix()
        _check(lib().qmr_matrix_load(gpu.handle, self._h, name.encode(), rows, cols, C.byref(m)))
        own = lambda h: Buffer(h) if h else None  # the Buffer objects release them
        return Matrix(own(m.weight), own(m.scales), own(m.biases), m.rows, m.cols, m.bits,
                      m.group, bool(m.metadata_bf16))

    def close(self) -> None:
        if self._h:
            lib().qmr_checkpoint_close(self._h)
            self._h = C.c_void_p()

    def __enter__(self) -> "Checkpoint":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        if _alive:
            try:
                self.close()
            except Exception:
                pass

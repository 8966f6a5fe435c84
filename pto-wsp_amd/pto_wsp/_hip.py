"""ctypes binding of libptowsp_hip.so (the C ABI in include/ptowsp_hip.h).

This is the only way the Python API reaches the GPU: there is no CPU
fallback.  If the library has not been built, importing this module raises.
``torch`` is imported first so that the library binds to the HIP runtime
torch already loaded (one runtime per process); torch is otherwise only used
to accept device-resident ``torch.Tensor`` data and the current stream.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

try:  # one HIP runtime per process: let torch load it first when present
    import torch
except ImportError:  # pragma: no cover - torch is part of this image
    torch = None

from pto_wsp.types import DType, Tensor

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libptowsp_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"libptowsp_hip.so not found at {LIB_PATH}; build it with `python -c \"import __graft_entry__ as g; g.build()\"`"
        " (the HIP target has no CPU fallback)")

_lib = ctypes.CDLL(LIB_PATH)


class RunInfo(ctypes.Structure):
    _fields_ = [("total_cycles", ctypes.c_uint64), ("task_count", ctypes.c_uint64),
                ("launches", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class Timing(ctypes.Structure):
    _fields_ = [("device_ms", ctypes.c_double), ("h2d_ms", ctypes.c_double), ("d2h_ms", ctypes.c_double)]


_vp = ctypes.c_void_p
_lib.ptowsp_hip_compile.argtypes = [ctypes.c_char_p, ctypes.POINTER(_vp)]
_lib.ptowsp_hip_compile.restype = ctypes.c_int
_lib.ptowsp_hip_launch.argtypes = [_vp, _vp, _vp, ctypes.POINTER(RunInfo)]
_lib.ptowsp_hip_launch.restype = ctypes.c_int
_lib.ptowsp_hip_synchronize.argtypes = [_vp, ctypes.POINTER(Timing)]
_lib.ptowsp_hip_synchronize.restype = ctypes.c_int
_lib.ptowsp_hip_workload_main.argtypes = [_vp, _vp, _vp]
_lib.ptowsp_hip_workload_main.restype = ctypes.c_uint64
_lib.ptowsp_hip_last_error.restype = ctypes.c_char_p
_lib.ptowsp_hip_release.argtypes = [_vp]
_lib.ptowsp_hip_num_launches.argtypes = [_vp]
_lib.ptowsp_hip_kernel_cycles.argtypes = [_vp, ctypes.c_char_p]
_lib.ptowsp_hip_kernel_cycles.restype = ctypes.c_uint64
_lib.ptowsp_hip_kernel_family.argtypes = [_vp, ctypes.c_char_p]
_lib.ptowsp_hip_run_result.argtypes = [_vp, ctypes.POINTER(RunInfo)]
_lib.ptowsp_hip_run_result.restype = ctypes.c_int
_lib.ptowsp_hip_precompile.argtypes = [_vp, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]
_lib.ptowsp_hip_precompile.restype = ctypes.c_int
_lib.ptowsp_hip_cycle_model.argtypes = [_vp, _vp, ctypes.POINTER(RunInfo)]
_lib.ptowsp_hip_cycle_model.restype = ctypes.c_int
_lib.ptowsp_rt_create.restype = _vp
_lib.ptowsp_rt_destroy.argtypes = [_vp]
_lib.ptowsp_rt_set_tensor.argtypes = [_vp, ctypes.c_uint32, _vp, ctypes.c_uint32, ctypes.POINTER(ctypes.c_int64)]
_lib.ptowsp_rt_set_axis_size.argtypes = [_vp, ctypes.c_char_p, ctypes.c_int64]
_lib.ptowsp_rt_set_symbol_u64.argtypes = [_vp, ctypes.c_uint64, ctypes.c_uint64]
_lib.ptowsp_rt_set_symbol_ptr.argtypes = [_vp, ctypes.c_uint64, _vp]
_lib.ptowsp_rt_clear.argtypes = [_vp]
_lib.ptowsp_rt_reset_slots.argtypes = [_vp]
_lib.ptowsp_rt_reset_slots.restype = ctypes.c_int
_lib.ptowsp_rt_context.argtypes = [_vp]
_lib.ptowsp_rt_context.restype = _vp

FAMILIES = {0: "row_program", 1: "tile_program", 2: "gemm", 3: "decode", 4: "custom"}

_NUMPY_DTYPES = {
    DType.F32: np.float32, DType.F16: np.float16, DType.BF16: np.uint16, DType.F64: np.float64,
    DType.I8: np.int8, DType.I16: np.int16, DType.I32: np.int32, DType.I64: np.int64,
    DType.U8: np.uint8, DType.U16: np.uint16, DType.U32: np.uint32, DType.U64: np.uint64,
}


def _torch_dtypes():
    if torch is None:
        return {}
    return {DType.F32: torch.float32, DType.F16: torch.float16, DType.BF16: torch.bfloat16,
            DType.F64: torch.float64, DType.I8: torch.int8, DType.I16: torch.int16, DType.I32: torch.int32,
            DType.I64: torch.int64, DType.U8: torch.uint8}


def _error() -> str:
    return _lib.ptowsp_hip_last_error().decode(errors="replace")


def tensor_binding(t: Tensor):
    """(pointer, element strides, keep-alive object, is_cuda) of a base tensor's storage."""
    d = t.data
    if d is None:
        dt = _NUMPY_DTYPES.get(t.dtype)
        if dt is None:
            raise ValueError(f"Unsupported dtype for codegen runtime: {t.dtype}")
        t.data = d = np.zeros(t.shape, dtype=dt)
    if isinstance(d, np.ndarray):
        want = _NUMPY_DTYPES.get(t.dtype)
        if want is None or d.dtype != np.dtype(want):
            raise TypeError(f"tensor of dtype {t.dtype.value} holds a numpy {d.dtype} array")
        if tuple(d.shape) != tuple(t.shape):
            raise ValueError(f"tensor shape {t.shape} does not match its data {d.shape}")
        strides = [s // d.itemsize for s in d.strides]
        if any(s * d.itemsize != b for s, b in zip(strides, d.strides)):
            raise ValueError("numpy strides must be multiples of the item size")
        return d.ctypes.data, strides, d, False
    if torch is not None and isinstance(d, torch.Tensor):
        want = _torch_dtypes().get(t.dtype)
        if d.dtype != want:
            raise TypeError(f"tensor of dtype {t.dtype.value} holds a torch {d.dtype} tensor")
        if tuple(d.shape) != tuple(t.shape):
            raise ValueError(f"tensor shape {t.shape} does not match its data {tuple(d.shape)}")
        return d.data_ptr(), list(d.stride()), d, d.is_cuda
    raise TypeError(f"Tensor.data must be a numpy array or a torch tensor (got {type(d).__name__})")


@dataclass
class LaunchResult:
    total_cycles: int
    task_count: int
    launches: int


@dataclass
class SyncTiming:
    device_ms: float
    h2d_ms: float
    d2h_ms: float


class NativeProgram:
    """A compiled module in libptowsp_hip.so."""

    def __init__(self, module_text: str) -> None:
        h = _vp()
        if _lib.ptowsp_hip_compile(module_text.encode(), ctypes.byref(h)) != 0:
            raise RuntimeError(_error())
        self._h = h
        self._rt = _vp(_lib.ptowsp_rt_create())
        self._live: list = []

    def __del__(self) -> None:
        lib = globals().get("_lib")
        if lib is None:
            return
        if getattr(self, "_h", None):
            lib.ptowsp_hip_release(self._h)
            self._h = None
        if getattr(self, "_rt", None):
            lib.ptowsp_rt_destroy(self._rt)
            self._rt = None

    def num_launches(self) -> int:
        return int(_lib.ptowsp_hip_num_launches(self._h))

    def kernel_cycles(self, name: str) -> int:
        return int(_lib.ptowsp_hip_kernel_cycles(self._h, name.encode()))

    def kernel_family(self, name: str) -> str:
        return FAMILIES.get(int(_lib.ptowsp_hip_kernel_family(self._h, name.encode())), "unknown")

    def precompile(self, index: int = 0, serial: bool = False, merged: bool = False, pingpong: bool = False,
                   seq_mask: int = 0, row_loops: bool = False, decode_norm: bool = False) -> str:
        """Emits and builds every launch; returns the source of launch `index`.

        serial: the in-order variant used when grid tasks overlap, with seq_mask the grid
        variables (bit v) looped in program order inside each workgroup, one group of tasks per
        workgroup (0: all of them in one workgroup); row_loops: row-program launches whose in-kernel
        loops run inside each row's lane team;
        merged: GEMM launches with the last two grid loops merged 2x2 per block;
        pingpong: merged 128x128 tasks with K step 32 / 64 as the two-group
        ping-pong block; decode_norm: decode launches with the following `out = o / l`
        launch folded in (the form a run uses when that launch follows).
        """
        src = ctypes.c_char_p()
        flags = ((1 if serial else 0) | (2 if merged else 0) | (4 if pingpong else 0) | (16 if row_loops else 0)
                 | (32 if decode_norm else 0) | ((int(seq_mask) & 0xFF) << 8))
        if _lib.ptowsp_hip_precompile(self._h, int(index), flags, ctypes.byref(src)) != 0:
            raise RuntimeError(_error())
        return src.value.decode() if src.value else ""

    def _bind_key(self, tensors, axis_sizes, symbols_u64, symbols_ptr):
        """Identity of a binding made only of device-resident torch tensors (storage pointer and
        strides per tensor, plus the axis sizes and symbols), or None when any tensor is host
        memory (those are staged through HBM on every launch)."""
        if torch is None:
            return None
        key = []
        for t in tensors:
            d = t.data
            if not isinstance(d, torch.Tensor) or not d.is_cuda:
                return None
            key.append((id(d), d.data_ptr(), d.stride()))
        key.append(tuple(axis_sizes.items()))
        key.append(tuple(symbols_u64.items()))
        for k, v in symbols_ptr.items():
            # Only arrays bound as they are (read in place at every launch) can be cached; any
            # other value is copied to an int32 array at binding time.
            if not isinstance(v, np.ndarray) or v.dtype != np.int32 or not v.flags.c_contiguous:
                return None
            key.append((k, id(v), v.ctypes.data))
        return tuple(key)

    def _bind(self, tensors, axis_sizes, symbols_u64, symbols_ptr):
        key = self._bind_key(tensors, axis_sizes, symbols_u64, symbols_ptr)
        if key is not None and key == getattr(self, "_last_bind", None):
            return self._last_live, True
        self._last_bind = None
        _lib.ptowsp_rt_clear(self._rt)
        live = []
        any_cuda = False
        for tid, t in enumerate(tensors):
            ptr, strides, keep, is_cuda = tensor_binding(t)
            any_cuda |= is_cuda
            live.append(keep)
            arr = (ctypes.c_int64 * max(1, len(strides)))(*strides)
            _lib.ptowsp_rt_set_tensor(self._rt, tid, ptr, len(strides), arr)
        for name, v in axis_sizes.items():
            _lib.ptowsp_rt_set_axis_size(self._rt, str(name).encode(), int(v))
        for sid, v in symbols_u64.items():
            _lib.ptowsp_rt_set_symbol_u64(self._rt, int(sid), int(v) & 0xFFFFFFFFFFFFFFFF)
        for sid, a in symbols_ptr.items():
            arr = np.ascontiguousarray(a, dtype=np.int32)
            live.append(arr)
            _lib.ptowsp_rt_set_symbol_ptr(self._rt, int(sid), arr.ctypes.data)
        if key is not None:
            self._last_bind, self._last_live = key, live
        return live, any_cuda

    def launch(self, tensors, axis_sizes: dict, symbols_u64: dict, symbols_ptr: dict, stream=None) -> LaunchResult:
        live, any_cuda = self._bind(tensors, axis_sizes, symbols_u64, symbols_ptr)
        if stream is None and any_cuda and torch is not None:
            stream = torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice())
        info = RunInfo()
        _lib.ptowsp_rt_reset_slots(self._rt)  # every run starts with zeroed slots
        ctx = _lib.ptowsp_rt_context(self._rt)
        if _lib.ptowsp_hip_launch(self._h, ctx, _vp(stream) if stream else None, ctypes.byref(info)) != 0:
            raise RuntimeError(_error())
        self._live = live
        return LaunchResult(int(info.total_cycles), int(info.task_count), int(info.launches))

    def cycle_model(self, tensors, axis_sizes: dict, symbols_u64: dict, symbols_ptr: dict) -> LaunchResult:
        """Evaluate only the cycle model (host only, no launch)."""
        live, _ = self._bind(tensors, axis_sizes, symbols_u64, symbols_ptr)
        info = RunInfo()
        _lib.ptowsp_rt_reset_slots(self._rt)
        rc = _lib.ptowsp_hip_cycle_model(self._h, _lib.ptowsp_rt_context(self._rt), ctypes.byref(info))
        del live
        if rc != 0:
            raise RuntimeError(_error())
        return LaunchResult(int(info.total_cycles), int(info.task_count), 0)

    def run_result(self) -> LaunchResult:
        """Cycle model result of the last synchronized run."""
        info = RunInfo()
        if _lib.ptowsp_hip_run_result(self._h, ctypes.byref(info)) != 0:
            raise RuntimeError(_error())
        return LaunchResult(int(info.total_cycles), int(info.task_count), int(info.launches))

    def synchronize(self) -> SyncTiming:
        tm = Timing()
        try:
            if _lib.ptowsp_hip_synchronize(self._h, ctypes.byref(tm)) != 0:
                raise RuntimeError(_error())
        finally:
            self._live = []
        return SyncTiming(tm.device_ms, tm.h2d_ms, tm.d2h_ms)


def library():
    """The loaded ctypes library (for tests of the C ABI)."""
    return _lib

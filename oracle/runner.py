"""ctypes driver for the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker.  It plays the part of the reference's loader
(``CodegenRuntime`` + ``CodegenExecutable.run_with_symbols``,
src/python/pto_codegen.cpp:3453-3576): it binds numpy arrays, axis sizes,
symbols and 256 zeroed slots into a ``RuntimeContext`` and calls the oracle's
entry point.  ``run_workload`` mirrors ``Program.execute()+synchronize()`` for
target "cpu_sim" (python/pto_wsp/program.py:670-743).
"""

from __future__ import annotations

import ctypes
import os
import struct
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libptowsp_cpusim.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.pto_cpusim_run.argtypes = [ctypes.c_char_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64)]
        lib.pto_cpusim_run.restype = ctypes.c_int
        lib.pto_cpusim_last_error.restype = ctypes.c_char_p
        lib.pto_cpusim_last_task_count.restype = ctypes.c_uint64
        lib.pto_cpusim_eval_scalar.argtypes = [ctypes.c_char_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64),
                                               ctypes.POINTER(ctypes.c_char)]
        lib.pto_cpusim_eval_scalar.restype = ctypes.c_int
        _lib = lib
    return _lib


_AXIS = ctypes.CFUNCTYPE(ctypes.c_int64, ctypes.c_void_p, ctypes.c_char_p)
_SYMU = ctypes.CFUNCTYPE(ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64)
_SYMP = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64)
_SLOTG = ctypes.CFUNCTYPE(ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint32)
_SLOTS = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64)
_TPTR = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32)
_TSTR = ctypes.CFUNCTYPE(ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32)
_KERN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32)


class _RuntimeContext(ctypes.Structure):
    _fields_ = [
        ("get_axis_size", _AXIS),
        ("get_symbol_u64", _SYMU),
        ("get_symbol_ptr", _SYMP),
        ("get_slot_u64", _SLOTG),
        ("set_slot_u64", _SLOTS),
        ("get_tensor_ptr", _TPTR),
        ("get_tensor_stride", _TSTR),
        ("get_kernel", _KERN),
        ("ctx", ctypes.c_void_p),
    ]


def fnv1a_64(s: str) -> int:
    h = 0xCBF29CE484222325
    for b in s.encode("utf-8"):
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


@dataclass
class OracleResult:
    total_cycles: int
    task_count: int


_CUSTOM_WRAPPER = r"""// A cpp_src body wrapped the way the reference wraps it for its cpu_sim
// artifact (src/python/pto_codegen.cpp:3294-3324), with pto::cpu_sim's
// cycle counter restated as a thread-local.
#include <cstddef>
#include <cstdint>
#include "ptowsp_abi.h"
namespace pto { namespace cpu_sim {
static thread_local uint64_t g_cycles = 0;
inline void reset_cycles() { g_cycles = 0; }
inline void add_cycles(uint64_t n) { g_cycles += n; }
inline uint64_t read_cycles() { return g_cycles; }
} }
extern "C" uint64_t ptowsp_oracle_custom(const KernelTaskDesc* task, CSPTContext* cspt) {
  (void)task;
  (void)cspt;
  uint64_t cycles = 0;
#if defined(__CPU_SIM)
  pto::cpu_sim::reset_cycles();
#endif
@BODY@
#if defined(__CPU_SIM)
  if (cycles == 0) cycles = pto::cpu_sim::read_cycles();
#endif
  return cycles;
}
"""
_custom_cache: dict = {}


def _decode(tok: str) -> str:
    if tok == "%":
        return ""
    out, i = bytearray(), 0
    while i < len(tok):
        if tok[i] == "%" and i + 3 <= len(tok) and all(c in "0123456789ABCDEFabcdef" for c in tok[i + 1:i + 3]):
            out.append(int(tok[i + 1:i + 3], 16))
            i += 3
        else:
            out += tok[i].encode()
            i += 1
    return out.decode("utf-8")


def custom_kernels(module_text: str) -> dict:
    """{kernel index: (library, function address)} for the module's custom kernels, each
    compiled with g++ into oracle/_build/custom/ (cached by content): a cpp_src body inside
    the reference's wrapper (entry ptowsp_oracle_custom), or a cpp_tu_path translation unit
    as it is, against the ABI headers in oracle/abi/ (entry: the kernel's name, the symbol
    the reference's workload loop calls, src/python/pto_codegen.cpp:2645-2651)."""
    import hashlib

    out = {}
    kidx = 0
    for line in module_text.splitlines():
        toks = line.split()
        if not toks or toks[0] != "K":
            continue
        if len(toks) > 6 and toks[5] in ("1", "2"):
            tu = toks[5] == "2"
            src = _decode(toks[6]) if tu else _CUSTOM_WRAPPER.replace("@BODY@", _decode(toks[6]))
            entry = _decode(toks[1]) if tu else "ptowsp_oracle_custom"
            key = hashlib.sha1((entry + "\n" + src).encode()).hexdigest()[:16]
            if key not in _custom_cache:
                d = os.path.join(_HERE, "_build", "custom")
                os.makedirs(d, exist_ok=True)
                cpp, so = os.path.join(d, f"k_{key}.cpp"), os.path.join(d, f"k_{key}.so")
                if not os.path.exists(so):
                    open(cpp, "w").write(src)
                    subprocess.run(["g++", "-std=c++17", "-O1", "-D__CPU_SIM=1", "-shared", "-fPIC",
                                    "-I", os.path.join(os.path.dirname(_HERE), "include"),
                                    "-I", os.path.join(_HERE, "abi"), cpp, "-o", so + ".tmp"], check=True)
                    os.replace(so + ".tmp", so)
                lib = ctypes.CDLL(so)
                _custom_cache[key] = (lib, ctypes.cast(getattr(lib, entry), ctypes.c_void_p).value)
            out[kidx] = _custom_cache[key]
        kidx += 1
    return out


def run_module(module_text: str, arrays: list, axis_sizes: dict | None = None,
               symbols_u64: dict | None = None, symbols_ptr: dict | None = None) -> OracleResult:
    """Run a serialized module on host numpy arrays (modified in place)."""
    lib = _load()
    arrays = list(arrays)
    for a in arrays:
        if not isinstance(a, np.ndarray):
            raise TypeError(f"oracle tensors must be numpy arrays (got {type(a).__name__})")
    axis_sizes = {str(k): int(v) for k, v in (axis_sizes or {}).items()}
    symbols_u64 = dict(symbols_u64 or {})
    symbols_ptr = dict(symbols_ptr or {})
    slots = [0] * 256

    def get_axis_size(_ctx, name):
        return axis_sizes.get(name.decode(), 0)

    def get_symbol_u64(_ctx, sid):
        return symbols_u64.get(int(sid), 0) & 0xFFFFFFFFFFFFFFFF

    def get_symbol_ptr(_ctx, sid):
        a = symbols_ptr.get(int(sid))
        return None if a is None else a.ctypes.data

    def get_slot(_ctx, i):
        return slots[i] if i < 256 else 0

    def set_slot(_ctx, i, v):
        if i < 256:
            slots[i] = v

    def get_tensor_ptr(_ctx, tid):
        return arrays[tid].ctypes.data if tid < len(arrays) else None

    def get_tensor_stride(_ctx, tid, dim):
        if tid >= len(arrays) or dim >= arrays[tid].ndim:
            return 0
        a = arrays[tid]
        return (a.strides[dim] // a.itemsize) & 0xFFFFFFFFFFFFFFFF

    kernels = custom_kernels(module_text)

    def get_kernel(_ctx, k):
        return kernels[k][1] if k in kernels else None

    cbs = (_AXIS(get_axis_size), _SYMU(get_symbol_u64), _SYMP(get_symbol_ptr), _SLOTG(get_slot),
           _SLOTS(set_slot), _TPTR(get_tensor_ptr), _TSTR(get_tensor_stride), _KERN(get_kernel))
    rc = _RuntimeContext(*cbs, None)
    cycles = ctypes.c_uint64(0)
    status = lib.pto_cpusim_run(module_text.encode(), ctypes.byref(rc), ctypes.byref(cycles))
    if status != 0:
        raise RuntimeError("cpu_sim oracle: " + lib.pto_cpusim_last_error().decode(errors="replace"))
    return OracleResult(int(cycles.value), int(lib.pto_cpusim_last_task_count()))


def _host_array(t) -> np.ndarray:
    from pto_wsp.types import DType

    d = t.data
    if d is None:
        dt = {DType.F32: np.float32, DType.F16: np.float16, DType.BF16: np.uint16,
              DType.I32: np.int32, DType.I64: np.int64}.get(t.dtype)
        if dt is None:
            raise ValueError(f"Unsupported dtype for the oracle: {t.dtype}")
        t.data = np.zeros(t.shape, dtype=dt)
        return t.data
    if isinstance(d, np.ndarray):
        return d
    raise TypeError(f"oracle runs on numpy-backed tensors (got {type(d).__name__})")


def run_workload(workload, axis_sizes: dict | None = None, symbols_u64: dict | None = None,
                 symbols_ptr: dict | None = None, module_name: str | None = None) -> OracleResult:
    """Serialize ``workload`` with the product's bridge and run it on the oracle.

    Tensors must hold numpy arrays; outputs are written in place, exactly as
    the reference's cpu_sim target writes into its numpy buffers.
    """
    from pto_wsp.ir_bridge import workload_to_codegen_ir
    from pto_wsp.program import Program

    name = module_name or (workload._name or "main")
    build = workload_to_codegen_ir(workload, module_name=name)
    arrays = [_host_array(t) for t in build.tensors]
    sizes = Program._infer_axis_sizes(workload)
    sizes.update(axis_sizes or {})
    return run_module(build.module, arrays, sizes, symbols_u64, symbols_ptr)


def eval_scalar(expr_text: str, symbols_u64: dict | None = None, slots: list | None = None) -> tuple[str, int]:
    """(C type code, value bits) of one scalar expression in the module's token form."""
    lib = _load()
    symbols_u64 = dict(symbols_u64 or {})
    slots = list(slots or [0] * 256)

    def get_symbol_u64(_ctx, sid):
        return symbols_u64.get(int(sid), 0) & 0xFFFFFFFFFFFFFFFF

    def get_slot(_ctx, i):
        return slots[i] if i < len(slots) else 0

    cbs = (_AXIS(lambda _c, _n: 0), _SYMU(get_symbol_u64), _SYMP(lambda _c, _s: None), _SLOTG(get_slot),
           _SLOTS(lambda _c, _i, _v: None), _TPTR(lambda _c, _t: None), _TSTR(lambda _c, _t, _d: 0),
           _KERN(lambda _c, _k: None))
    rc = _RuntimeContext(*cbs, None)
    value, typ = ctypes.c_uint64(0), ctypes.c_char(b"?")
    if lib.pto_cpusim_eval_scalar(expr_text.encode(), ctypes.byref(rc), ctypes.byref(value), ctypes.byref(typ)) != 0:
        raise RuntimeError("cpu_sim oracle: " + lib.pto_cpusim_last_error().decode(errors="replace"))
    return typ.value.decode(), int(value.value)


def f32_symbol(value: float) -> int:
    return struct.unpack("<I", struct.pack("<f", float(value)))[0]

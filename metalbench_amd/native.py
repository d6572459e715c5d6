"""ctypes binding of libmbhip.so (the C ABI declared in include/mbhip.h).

This is the in-process replacement of the reference's host-binary boundary
(reference mlx/scripts/harness.py:36-49 `_run_host`, metal/scripts/main.mm:73-197):
instead of a JSON manifest and .bin files, the harness passes device pointers
of caller-owned buffers through `mb_run`.

There is no fallback: if the library is missing or a call fails, a
`NativeError` is raised with the library's own message.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import (POINTER, Structure, Union, byref, c_char, c_char_p, c_double,
                    c_float, c_int, c_int32, c_uint16, c_uint32, c_uint64, c_void_p)
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "lib" / "libmbhip.so"

MB_OK = 0
ERROR_NAMES = {
    -1: "MB_E_NO_DEVICE", -2: "MB_E_NOT_FOUND", -3: "MB_E_BINDING", -4: "MB_E_DTYPE",
    -5: "MB_E_HIP", -6: "MB_E_STATE", -7: "MB_E_ARG",
}

ROLE_INPUT, ROLE_OUTPUT, ROLE_SCALAR = 0, 1, 2
DTYPE_CODE = {"f32": 0, "f16": 1, "i32": 2, "u32": 3, "bf16": 4}

RUN_SYNC_EACH = 0
RUN_PIPELINED = 1
RUN_PARTS = 2
RUN_WALL_ONLY = 4
RUN_COLD = 8
MAX_PARTS = 8


class NativeError(RuntimeError):
    """A libmbhip.so call returned an error code."""

    def __init__(self, call: str, code: int, message: str):
        self.code = code
        super().__init__(f"{call} failed: {ERROR_NAMES.get(code, code)}: {message}")


class _Scalar(Union):
    _fields_ = [("u32", c_uint32), ("i32", c_int32), ("f32", c_float)]


class MbBinding(Structure):
    _fields_ = [("index", c_uint32), ("role", c_uint32), ("dev_ptr", c_void_p),
                ("nbytes", c_uint64), ("dtype", c_uint32), ("_pad", c_uint32),
                ("scalar", _Scalar), ("_pad2", c_uint32)]


class MbTiming(Structure):
    _fields_ = [("min_ms", c_double), ("median_ms", c_double), ("mean_ms", c_double),
                ("iters", c_int32), ("n_parts", c_int32),
                ("part_median_ms", c_double * MAX_PARTS),
                ("part_mean_ms", c_double * MAX_PARTS),
                ("part_names", (c_char * 48) * MAX_PARTS),
                ("wall_ms", c_double)]


class MbDeviceInfo(Structure):
    _fields_ = [("name", c_char * 256), ("arch", c_char * 64), ("ordinal", c_int32),
                ("cu_count", c_int32), ("clock_khz", c_int32), ("mem_clock_khz", c_int32),
                ("mem_bus_width", c_int32), ("warp_size", c_int32), ("hbm_bytes", c_uint64),
                ("lds_per_block", c_uint64), ("lds_per_cu", c_uint64), ("l2_bytes", c_uint64),
                ("max_threads_per_block", c_int32), ("regs_per_block", c_int32)]


class MbKernelAttrs(Structure):
    _fields_ = [("static_lds_bytes", c_uint64), ("max_threads_per_block", c_int32),
                ("num_regs", c_int32), ("private_bytes", c_uint64), ("n_parts", c_int32),
                ("dominant_part", c_int32), ("arch_vgprs", c_int32), ("agprs", c_int32),
                ("sgprs", c_int32), ("waves_per_simd", c_int32)]


class MbDecoderStepArgs(Structure):
    _fields_ = [("batch", c_uint32), ("d_model", c_uint32), ("n_heads", c_uint32),
                ("n_kv_heads", c_uint32), ("head_dim", c_uint32), ("d_ff", c_uint32),
                ("cache_len", c_uint32), ("cache_stride", c_uint32),
                ("rope_base", c_float), ("eps", c_float),
                ("x", c_void_p), ("w_qkv", c_void_p), ("w_o", c_void_p), ("w_gu", c_void_p),
                ("w_down", c_void_p), ("k_cache", c_void_p), ("v_cache", c_void_p),
                ("y", c_void_p), ("k_new", c_void_p), ("v_new", c_void_p),
                ("workspace", c_void_p), ("workspace_bytes", c_uint64)]


STRUCTS = {0: MbBinding, 1: MbTiming, 2: MbDeviceInfo, 3: MbKernelAttrs, 4: MbDecoderStepArgs}

# Every exported function: name -> (restype, argtypes).
SIGNATURES = {
    "mb_abi_version": (c_int, []),
    "mb_abi_struct_size": (c_int, [c_int]),
    "mb_init": (c_int, [c_int]),
    "mb_shutdown": (c_int, []),
    "mb_last_error": (c_char_p, []),
    "mb_device_info_get": (c_int, [POINTER(MbDeviceInfo)]),
    "mb_set_stream": (c_int, [c_void_p]),
    "mb_kernel_count": (c_int, []),
    "mb_kernel_name": (c_char_p, [c_int]),
    "mb_kernel_find": (c_int, [c_char_p, POINTER(c_int)]),
    "mb_kernel_attrs_get": (c_int, [c_int, POINTER(MbKernelAttrs)]),
    "mb_run": (c_int, [c_int, POINTER(MbBinding), c_int, c_int, c_int, c_uint32,
                       POINTER(MbTiming)]),
    "mb_launch_transpose_2d_f32": (c_int, [c_void_p, c_void_p, c_uint32, c_uint32, c_void_p]),
    "mb_launch_matmul_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32,
                                     c_uint32, c_void_p]),
    "mb_launch_matmul_bf16": (c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32,
                                      c_uint32, c_void_p]),
    "mb_launch_conv2d_nhwc_f32": (c_int, [c_void_p, c_void_p, c_void_p] + [c_uint32] * 9
                                  + [c_void_p]),
    "mb_decoder_step_workspace_bytes": (c_uint64, [POINTER(MbDecoderStepArgs)]),
    "mb_launch_llama_decoder_step_bf16": (c_int, [POINTER(MbDecoderStepArgs), c_void_p]),
    "mb_launch_llama_decoder_step_bf16_noalloc": (c_int, [POINTER(MbDecoderStepArgs), c_void_p]),
    "mb_launch_copy_f32": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p]),
}

_lib = None


def library_path() -> Path:
    return Path(os.environ.get("MBHIP_LIB", LIB_PATH))


def load() -> ctypes.CDLL:
    """Load libmbhip.so (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    # torch ships its own HIP runtime whose soname (libamdhip64.so.7) is the one
    # libmbhip.so links against: loading torch first makes both share one
    # runtime, so torch-allocated device pointers are valid in the library.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    path = library_path()
    if not path.is_file():
        raise NativeError("load", -6, f"{path} not found; build it with `make` "
                          "or __graft_entry__.build()")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)   # AttributeError if the symbol is missing
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().mb_last_error().decode(errors="replace")


def check(call: str, rc: int) -> None:
    if rc != MB_OK:
        raise NativeError(call, rc, last_error())


_initialized = False


def init(ordinal: int = 0) -> None:
    """mb_init(ordinal); idempotent."""
    global _initialized
    if _initialized:
        return
    check("mb_init", load().mb_init(ordinal))
    _initialized = True


def shutdown() -> None:
    global _initialized
    if _lib is not None:
        _lib.mb_shutdown()
    _initialized = False


def device_info() -> dict:
    init()
    info = MbDeviceInfo()
    check("mb_device_info_get", load().mb_device_info_get(byref(info)))
    out = {}
    for name, _ in MbDeviceInfo._fields_:
        v = getattr(info, name)
        out[name] = v.decode(errors="replace") if isinstance(v, bytes) else v
    return out


def kernel_names() -> list[str]:
    lib = load()
    return [lib.mb_kernel_name(i).decode() for i in range(lib.mb_kernel_count())]


def kernel_find(function: str) -> int:
    kid = c_int(-1)
    check("mb_kernel_find", load().mb_kernel_find(function.encode(), byref(kid)))
    return kid.value


def kernel_attrs(kid: int) -> dict:
    init()
    a = MbKernelAttrs()
    check("mb_kernel_attrs_get", load().mb_kernel_attrs_get(kid, byref(a)))
    return {name: getattr(a, name) for name, _ in MbKernelAttrs._fields_}


def make_binding(index: int, role: int, dtype: str, dev_ptr: int = 0, nbytes: int = 0,
                 value=None) -> MbBinding:
    b = MbBinding()
    b.index = index
    b.role = role
    b.dtype = DTYPE_CODE[dtype]
    b.dev_ptr = dev_ptr or None
    b.nbytes = nbytes
    if role == ROLE_SCALAR:
        if dtype == "f32":
            b.scalar.f32 = float(value)
        elif dtype == "i32":
            b.scalar.i32 = int(value)
        else:
            b.scalar.u32 = int(value)
    return b


def run(kid: int, bindings: list[MbBinding], warmup: int, iters: int,
        flags: int = RUN_SYNC_EACH) -> dict:
    """mb_run: bind, warm up, time `iters` dispatches; returns the timing dict
    (the `{min_ms, median_ms, mean_ms, iters}` of reference main.mm:184-195)."""
    init()
    arr = (MbBinding * max(1, len(bindings)))(*bindings)
    t = MbTiming()
    check("mb_run", load().mb_run(kid, arr, len(bindings), warmup, iters, flags, byref(t)))
    out = {"min_ms": t.min_ms, "median_ms": t.median_ms, "mean_ms": t.mean_ms,
           "iters": t.iters, "wall_ms": t.wall_ms}
    if t.n_parts:
        out["parts"] = [
            {"name": t.part_names[i].value.decode(), "median_ms": t.part_median_ms[i],
             "mean_ms": t.part_mean_ms[i]}
            for i in range(t.n_parts)
        ]
    return out

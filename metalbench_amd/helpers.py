"""Registry loading, spec validation, seeded inputs and chip detection.

Mirrors reference mlx/scripts/mlx_helpers.py for the gfx950 backend:
  * `load_baseline(name)` resolves `mlx/kernels/<set>/<name>.py` (the `Model`
    spec) plus `REGISTRY[name]` (reference mlx_helpers.py:185-287);
  * `Output` / `Scalar` / `BaselineSpec` are the same pydantic schema
    (reference :92-140) with bf16 added to the dtype tags;
  * inputs come from one seeded torch CPU generator consumed in binding order
    (reference :241-251 draws mx.random.normal after mx.random.seed), using the
    registry's optional `input_init` / `input_dtypes` keys;
  * `chip_info()` describes the GPU from libmbhip.so's mb_device_info (reference
    :356-382 and metal/scripts/setup.cpp:116-136 read sysctl instead).
"""
from __future__ import annotations

import functools
import importlib.util
import math
import os
import re
from pathlib import Path
from typing import Tuple

import numpy as np
from pydantic import BaseModel, Field, ValidationError, field_validator

REPO_ROOT = Path(__file__).resolve().parents[1]
BASELINE_ROOT = REPO_ROOT / "mlx" / "kernels"
KERNEL_ROOT = Path(__file__).resolve().parent / "csrc"
RESULTS_ROOT = REPO_ROOT / "results"
SESSION_PATH = REPO_ROOT / "session.json"
SETS = ("common", "standard", "full")

DTYPE_NP = {"f32": np.float32, "f16": np.float16, "i32": np.int32, "u32": np.uint32,
            "bf16": np.uint16}
DTYPE_BYTES = {"f32": 4, "f16": 2, "i32": 4, "u32": 4, "bf16": 2}
_VALID_DTYPES = ("f32", "f16", "i32", "u32", "bf16")


def torch_dtype(tag: str):
    import torch
    return {"f32": torch.float32, "f16": torch.float16, "i32": torch.int32,
            "u32": torch.int32, "bf16": torch.bfloat16}[tag]


# ---- spec types (reference mlx_helpers.py:92-140) ----------------------------------

class Output(BaseModel):
    binding: int = Field(ge=0, lt=32)
    dtype: str
    shape: Tuple[int, ...]

    @field_validator("dtype")
    @classmethod
    def _ok(cls, v):
        if v not in _VALID_DTYPES:
            raise ValueError(f"dtype must be {_VALID_DTYPES}, got {v!r}")
        return v


class Scalar(BaseModel):
    binding: int = Field(ge=0, lt=32)
    dtype: str
    value: float | int

    @field_validator("dtype")
    @classmethod
    def _ok(cls, v):
        if v not in ("u32", "i32", "f32"):
            raise ValueError(f"scalar dtype must be u32|i32|f32, got {v!r}")
        return v


class BaselineSpec(BaseModel):
    name: str
    metal_function: str
    threadgroup: Tuple[int, int, int]
    input_bindings: Tuple[int, ...]
    outputs: list[Output]
    rtol: float = 1e-4
    atol: float = 1e-5
    best_for: Tuple[str, ...] = ()

    @field_validator("threadgroup")
    @classmethod
    def _tg_pos(cls, v):
        if any(x <= 0 for x in v):
            raise ValueError(f"threadgroup dims must be > 0, got {v}")
        return v

    @field_validator("input_bindings")
    @classmethod
    def _unique(cls, v):
        if len(set(v)) != len(v):
            raise ValueError(f"input_bindings must be unique, got {v}")
        return v


# ---- seeded inputs -------------------------------------------------------------------

def _validate_init(init) -> tuple:
    kind = init[0]
    if kind == "normal" and len(init) == 3 and init[2] >= 0:
        return tuple(init)
    if kind == "uniform" and len(init) == 3 and init[1] <= init[2]:
        return tuple(init)
    if kind == "kaiming_normal" and len(init) == 2 and init[1] > 0:
        return tuple(init)
    raise ValueError(f"bad input_init entry {init!r}")


def generate_input(gen, shape, init=("normal", 0.0, 1.0), dtype="f32"):
    """One input tensor (CPU) drawn from `gen`, then cast to `dtype` (bf16 by
    round-to-nearest-even, torch's float->bfloat16 conversion)."""
    import torch
    init = _validate_init(init)
    shape = tuple(int(s) for s in shape)
    if init[0] == "uniform":
        lo, hi = init[1], init[2]
        t = torch.rand(shape, generator=gen, dtype=torch.float32) * (hi - lo) + lo
    else:
        if init[0] == "kaiming_normal":
            mean, std = 0.0, math.sqrt(2.0 / init[1])
        else:
            mean, std = init[1], init[2]
        t = torch.randn(shape, generator=gen, dtype=torch.float32)
        if std != 1.0:
            t.mul_(std)
        if mean != 0.0:
            t.add_(mean)
    if dtype != "f32":
        t = t.to(torch_dtype(dtype))
    return t.contiguous()


def make_inputs_from_meta(meta: dict, seed: int):
    """All inputs of a registry entry, in binding order, from one generator."""
    import torch
    gen = torch.Generator().manual_seed(int(seed))
    shapes = meta.get("input_shapes") or [meta["output_shape"]]
    n = len(shapes)
    dtypes = meta.get("input_dtypes") or ["f32"] * n
    inits = meta.get("input_init") or [("normal", 0.0, 1.0)] * n
    if len(dtypes) != n or len(inits) != n:
        raise ValueError("input_dtypes / input_init must have one entry per input")
    return [generate_input(gen, s, i, d) for s, i, d in zip(shapes, inits, dtypes)]


# ---- registry + Model loading (reference mlx_helpers.py:185-287) -----------------------

def _find_baseline(name):
    for s in SETS:
        p = BASELINE_ROOT / s / f"{name}.py"
        if p.exists():
            return p, s
    raise FileNotFoundError(
        f"baseline not found: searched mlx/kernels/{{{','.join(SETS)}}}/{name}.py")


def load_registry(set_name: str) -> dict:
    path = BASELINE_ROOT / set_name / "registry.py"
    spec = importlib.util.spec_from_file_location(f"_mb_registry_{set_name}", path)
    if spec is None or spec.loader is None:
        raise ImportError(f"cannot load {path}")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.REGISTRY


def all_kernels() -> list[tuple[str, str]]:
    out = []
    for s in SETS:
        if (BASELINE_ROOT / s / "registry.py").is_file():
            out += [(s, k) for k in sorted(load_registry(s))]
    return out


class Baseline:
    """A loaded registry entry: spec, Model reference and metadata."""

    def __init__(self, name, set_name, module, meta, spec, scalars):
        self.name, self.set_name, self.module, self.meta = name, set_name, module, meta
        self._spec, self._scalars = spec, scalars
        Model = getattr(module, "Model")
        self._model = Model(**meta.get("model_kwargs", {}))

    metal_function = property(lambda self: self._spec.metal_function)
    threadgroup = property(lambda self: self._spec.threadgroup)
    input_bindings = property(lambda self: self._spec.input_bindings)
    outputs = property(lambda self: self._spec.outputs)
    rtol = property(lambda self: self._spec.rtol)
    atol = property(lambda self: self._spec.atol)
    best_for = property(lambda self: self._spec.best_for)
    compute_dtype = property(lambda self: self.meta.get("compute_dtype", "f32"))
    input_dtypes = property(lambda self: list(
        self.meta.get("input_dtypes") or ["f32"] * len(self.meta["input_shapes"])))

    def make_inputs(self, seed):
        return make_inputs_from_meta(self.meta, seed)

    def reference(self, *inputs):
        import torch
        with torch.no_grad():
            return self._model.forward(*inputs)

    def scalars(self, inputs=None):
        return list(self._scalars)

    def grid(self, inputs=None):
        return tuple(self.meta["grid"])

    def flops(self, inputs=None):
        v = self.meta.get("flops")
        return int(v) if v is not None else None

    def bytes(self, inputs=None):
        v = self.meta.get("bytes")
        return int(v) if v is not None else None


def load_baseline(name) -> Baseline:
    path, set_name = _find_baseline(name)
    mod_spec = importlib.util.spec_from_file_location(f"_mb_{name}", path)
    if mod_spec is None or mod_spec.loader is None:
        raise ImportError(f"cannot load {path}")
    mod = importlib.util.module_from_spec(mod_spec)
    mod_spec.loader.exec_module(mod)
    if getattr(mod, "Model", None) is None:
        raise AttributeError(f"{name}.py: missing Model class")

    meta = load_registry(set_name).get(name)
    if meta is None:
        raise KeyError(f"no registry entry for '{name}'")

    n_in = len(meta["input_shapes"])
    out_dtype = meta.get("output_dtype", "f32")
    raw_outputs = [dict(binding=n_in, dtype=out_dtype, shape=meta["output_shape"])]
    for i, extra in enumerate(meta.get("extra_outputs", [])):
        raw_outputs.append(dict(binding=n_in + 1 + i, dtype=extra.get("dtype", out_dtype),
                                shape=extra["shape"]))
    try:
        outputs = [Output(**o) for o in raw_outputs]
        scalars = [Scalar(**s) for s in meta["scalars"]]
        spec = BaselineSpec(
            name=name,
            metal_function=meta["metal_function"],
            threadgroup=tuple(meta["threadgroup"]),
            input_bindings=tuple(meta["input_bindings"]),
            outputs=outputs,
            rtol=meta.get("rtol", 1e-4),
            atol=meta.get("atol", 1e-5),
            best_for=tuple(meta.get("BEST_FOR", ())),
        )
    except ValidationError as e:
        raise ValueError(f"registry entry for '{name}' invalid:\n{e}") from e
    if len(spec.input_bindings) != n_in:
        raise ValueError(f"registry entry for '{name}': {n_in} input shapes but "
                         f"{len(spec.input_bindings)} input bindings")
    return Baseline(name, set_name, mod, meta, spec, scalars)


def build_manifest(b: Baseline, inputs, *, warmup, iters, chip_type=None, profile=False,
                   capture_host=None):
    """The dispatch description (reference mlx_helpers.py:290-335) without file
    paths: inputs and outputs are handed over as device buffers in-process.
    `capture_path` is present when a kernel trace of one dispatch is asked for
    (reference :333-334)."""
    buffers = []
    for binding, t, dt in zip(b.input_bindings, inputs, b.input_dtypes):
        buffers.append({"binding": int(binding), "role": "input", "dtype": dt,
                        "size": int(t.numel()) * DTYPE_BYTES[dt]})
    for o in b.outputs:
        buffers.append({"binding": int(o.binding), "role": "output", "dtype": o.dtype,
                        "size": int(np.prod(o.shape)) * DTYPE_BYTES[o.dtype]})
    for s in b.scalars(inputs):
        buffers.append({"binding": int(s.binding), "role": "scalar",
                        "dtype": s.dtype, "value": s.value})
    threadgroup = list(b.threadgroup)
    grid = list(b.grid(inputs))
    if chip_type:
        override = _get_chip_override(b.name, chip_type)
        if override:
            threadgroup = list(override.get("threadgroup", threadgroup))
            grid = list(override.get("grid", grid))
    manifest = {
        "function": b.metal_function,
        "library": "metalbench_amd/lib/libmbhip.so",
        "buffers": buffers,
        "grid": grid,
        "threadgroup": threadgroup,
        "warmup": int(warmup),
        "iters": int(iters),
        "profile": bool(profile),
    }
    if capture_host:
        manifest["capture_path"] = str(capture_host)
    return manifest


def find_kernel_source(name: str) -> Path | None:
    """The HIP source file that registers the kernel behind `name`'s
    `metal_function` (reference mlx_helpers.py:50-80 resolves .metal files)."""
    try:
        b = load_baseline(name)
        fn = b.metal_function
    except Exception:
        fn = name
    pat = re.compile(r'register_kernel\(\{\s*"' + re.escape(fn) + r'"')
    for p in sorted(KERNEL_ROOT.glob("*.hip")):
        if pat.search(p.read_text()):
            return p
    return None


# ---- chip detection (reference mlx_helpers.py:340-401, setup.cpp:116-136) --------------

def _host_ram_bytes() -> int:
    try:
        for line in Path("/proc/meminfo").read_text().splitlines():
            if line.startswith("MemTotal:"):
                return int(line.split()[1]) * 1024
    except Exception:
        pass
    return 0


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


@functools.lru_cache(maxsize=1)
def chip_info() -> dict:
    """GPU identity for result bucketing.  type = the gfx target ("gfx950"),
    bucket = sanitised device name, e.g. "amd-instinct-mi355x"."""
    cpu_cores = os.cpu_count() or 0
    try:
        from . import native
        d = native.device_info()
        name = d["name"] or "unknown"
        arch = d["arch"].split(":")[0]
        return {"type": arch or "unknown", "name": name, "bucket": bucket_key_from_name(name),
                "cpu_cores": cpu_cores, "gpu_cores": d["cu_count"],
                "ram_bytes": _host_ram_bytes(), "hbm_bytes": d["hbm_bytes"],
                "clock_khz": d["clock_khz"], "cpu_model": cpu_model()}
    except Exception as e:   # no GPU / library not built
        return {"type": "unknown", "name": "unknown", "bucket": "unknown",
                "cpu_cores": cpu_cores, "gpu_cores": 0, "ram_bytes": _host_ram_bytes(),
                "hbm_bytes": 0, "clock_khz": 0, "cpu_model": cpu_model(), "error": str(e)}


def _kfd_gfx_targets() -> list[str]:
    """gfx targets of the GPUs the kernel driver lists, read from the KFD
    topology in sysfs (no HIP call, so no device is initialised): a node's
    gfx_target_version 90500 is gfx950."""
    out = []
    try:
        for props in sorted(Path("/sys/class/kfd/kfd/topology/nodes").glob("*/properties")):
            for line in props.read_text().splitlines():
                key, _, val = line.partition(" ")
                if key == "gfx_target_version" and val.strip().isdigit() and int(val) > 0:
                    v = int(val)
                    out.append(f"gfx{v // 10000}{(v // 100) % 100:x}{v % 100:x}")
    except Exception:
        pass
    return out


def host_chip_info() -> dict:
    """chip_info() without touching the GPU, for the modes that make no GPU call
    (--mlx-only, --dry-run): the gfx target comes from the KFD topology, and
    the marketing name is not queried."""
    targets = _kfd_gfx_targets()
    arch = targets[0] if targets else "unknown"
    name = f"AMD {arch} (not queried)" if targets else "unknown"
    return {"type": arch, "name": name, "bucket": bucket_key_from_name(name),
            "cpu_cores": os.cpu_count() or 0, "gpu_cores": 0, "ram_bytes": _host_ram_bytes(),
            "hbm_bytes": 0, "clock_khz": 0, "cpu_model": cpu_model()}


def bucket_key_from_name(name):
    s = "".join((c.lower() if c.isalnum() else "-") for c in name)
    while "--" in s:
        s = s.replace("--", "-")
    return s.strip("-") or "unknown"


def bucket_key():
    return chip_info()["bucket"]


def chip_generation(chip_type: str) -> str:
    """Bare target family: 'gfx950' -> 'gfx950'; 'gfx942:sramecc+' -> 'gfx942'."""
    return chip_type.split(":")[0]


@functools.lru_cache(maxsize=1)
def _load_tuning() -> dict:
    spec = importlib.util.spec_from_file_location(
        "_mb_tuning", BASELINE_ROOT / "common" / "tuning.py")
    if spec is None or spec.loader is None:
        return {}
    mod = importlib.util.module_from_spec(spec)
    try:
        spec.loader.exec_module(mod)
        return getattr(mod, "CHIP_TUNING", {})
    except Exception:
        return {}


def _get_chip_override(name: str, chip_type: str) -> dict | None:
    tuning = _load_tuning()
    return tuning.get((name, chip_type)) or tuning.get((name, chip_generation(chip_type)))

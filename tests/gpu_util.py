"""Helpers for the GPU parity tests: seeded inputs, launches through the C ABI."""
from __future__ import annotations

import numpy as np
import torch

from metalbench_amd import helpers as H
from metalbench_amd import native


def seeded(seed: int, shape, init=("normal", 0.0, 1.0), dtype="f32"):
    gen = torch.Generator().manual_seed(seed)
    return H.generate_input(gen, shape, init, dtype)


def sync():
    torch.cuda.synchronize()


def launch(fn_name: str, *args):
    """Call an mb_launch_* entry point on the library stream and wait."""
    lib = native.load()
    rc = getattr(lib, fn_name)(*args)
    native.check(fn_name, rc)
    sync()


def ptr(t) -> int:
    return t.data_ptr()


def bits32(t) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int32).numpy()


def run_registry(name: str, seed: int = 0, warmup: int = 1, iters: int = 2, inputs=None):
    """Run a registry entry through mb_run (the harness path); returns
    (baseline, inputs, outputs, timing)."""
    from metalbench_amd import harness
    b = H.load_baseline(name)
    if inputs is None:
        inputs = b.make_inputs(seed)
    k_t, outs = harness._run_native(b, inputs, warmup, iters)
    return b, inputs, outs, k_t


def assert_close(actual, expected, rtol, atol, what=""):
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, (what, a.shape, e.shape)
    diff = np.abs(a - e)
    tol = atol + rtol * np.abs(e)
    bad = ~(diff <= tol)
    if bad.any():
        idx = np.unravel_index(np.argmax(np.where(bad, diff - tol, -np.inf)), a.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} / {a.size} elements out of tolerance "
                             f"(rtol={rtol}, atol={atol}); worst at {idx}: got {a[idx]!r}, "
                             f"expected {e[idx]!r}, max |diff| {diff.max():.3e}")


def run_bound(metal_function: str, inputs, outputs, scalars, dtype="f32"):
    """Run a registry kernel through mb_run with explicit bindings (shapes the
    registry does not hold).  inputs: [(binding, tensor)], outputs:
    [(binding, shape)], scalars: [(binding, dtype, value)].  Returns the
    outputs as CPU tensors."""
    native.init(0)
    dev = torch.device("cuda", 0)
    d_in = [(b, t.to(dev)) for b, t in inputs]
    d_out = [(b, torch.full(tuple(shape), float("nan"), dtype=torch.float32, device=dev))
             for b, shape in outputs]
    sync()
    binds = [native.make_binding(b, native.ROLE_INPUT, dtype, t.data_ptr(),
                                 t.numel() * t.element_size()) for b, t in d_in]
    binds += [native.make_binding(b, native.ROLE_OUTPUT, dtype, t.data_ptr(),
                                  t.numel() * t.element_size()) for b, t in d_out]
    binds += [native.make_binding(b, native.ROLE_SCALAR, dt, value=v) for b, dt, v in scalars]
    native.run(native.kernel_find(metal_function), binds, 0, 1, native.RUN_SYNC_EACH)
    sync()
    return [t.cpu() for _, t in d_out]

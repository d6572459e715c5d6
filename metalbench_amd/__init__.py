"""metalbench_amd — MI355X (gfx950) backend for MetalBench's kernel registry.

Layout:
  csrc/        hand-written HIP kernels + the C ABI runtime (libmbhip.so)
  lib/         the built libmbhip.so
  native.py    ctypes binding of include/mbhip.h
  helpers.py   registry / spec loading, seeded inputs, chip detection
  harness.py   evaluate + report + session persistence (`./bench <name>`)
  timing.py    CPU-baseline timer;  roofline.py  MI355X roofline
"""
__all__ = ["native", "helpers", "harness", "timing", "roofline"]

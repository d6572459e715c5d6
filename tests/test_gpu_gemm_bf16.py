"""bf16 GEMM (fp32 accumulate, bf16 out) on the GPU vs the float64 oracle.

Gate (benchmark configuration): rtol 1e-2 against the fp32-accumulated product, atol 1e-4.
Stronger check: with fp32 accumulation the error before rounding is ~1e-6
relative, far below half a bf16 ulp, so wherever |C| is not tiny (above 1% of
its RMS, where a bf16 ulp still dwarfs the fp32 accumulation noise) the
kernel's output must be the round-to-nearest-even bf16 of the exact product
within one bf16 ulp, and equal to it for almost every element."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close, launch, ptr, run_registry, seeded
from metalbench_amd import native

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _check_rounding(got_bits, exact, what, min_equal=0.99):
    want_bits = oracle.f32_to_bf16_bits(exact.astype(np.float32))
    # ordered distance in bf16 ulps (sign-magnitude -> two's complement)
    def ordered(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)
    ulps = np.abs(ordered(got_bits) - ordered(want_bits))
    ulps = ulps[np.abs(exact) >= 0.01 * np.sqrt(np.mean(exact * exact))]
    assert ulps.max() <= 1, f"{what}: max {ulps.max()} bf16 ulps off the rounded exact product"
    frac = float(np.mean(ulps == 0))
    assert frac >= min_equal, f"{what}: only {frac:.4f} of elements equal the rounded exact product"


@pytest.mark.parametrize("m,n,k", [
    (256, 256, 64), (512, 256, 128), (256, 512, 512), (300, 260, 72), (1, 8, 8), (17, 24, 40),
    (256, 256, 8), (513, 1000, 200), (5, 7, 3), (64, 300, 1000), (1024, 1024, 1024),
])
def test_matmul_bf16_shapes(mb, dev, m, n, k):
    a = seeded(m + 3 * k, (m, k), ("normal", 0.0, 0.02), "bf16")
    b = seeded(n + 5 * k, (k, n), ("normal", 0.0, 0.02), "bf16")
    d_a, d_b = a.to(dev), b.to(dev)
    d_c = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=dev)
    launch("mb_launch_matmul_bf16", ptr(d_a), ptr(d_b), ptr(d_c), m, n, k, None)
    exact = oracle.matmul(oracle.as_f64(a), oracle.as_f64(b))
    got = oracle.as_f64(d_c)
    assert_close(got, exact, 1e-2, 1e-4, f"matmul_bf16 {m}x{n}x{k}")
    _check_rounding(_bits(d_c), exact, f"matmul_bf16 {m}x{n}x{k}")


def _random_bf16_shapes(n, seed=71):
    """Seeded shapes: half ragged (guarded and element-wise kernels), half full
    256 x 256 tiles with K a multiple of 128 (the DMA kernel)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        if i % 2:
            out.append((256 * int(rng.integers(1, 4)), 256 * int(rng.integers(1, 4)),
                        128 * int(rng.integers(1, 7))))
        else:
            out.append(tuple(int(v) for v in rng.integers(1, 700, size=3)))
    return out


@pytest.mark.parametrize("m,n,k", _random_bf16_shapes(8))
def test_matmul_bf16_random_shapes(mb, dev, m, n, k):
    test_matmul_bf16_shapes(mb, dev, m, n, k)


def test_matmul_bf16_identity_exact(mb, dev):
    a = seeded(11, (256, 512), ("normal", 0.0, 1.0), "bf16")
    eye = torch.eye(512, dtype=torch.bfloat16)
    d_a, d_e = a.to(dev), eye.to(dev)
    d_c = torch.zeros((256, 512), dtype=torch.bfloat16, device=dev)
    launch("mb_launch_matmul_bf16", ptr(d_a), ptr(d_e), ptr(d_c), 256, 512, 512, None)
    assert torch.equal(d_c.cpu(), a)


def test_large_mm_registry_config_full(mb):
    """The 8192^3 config: all 67,108,864 outputs against the float64 product
    of the same bf16 operands (a few seconds of float64 BLAS on the host), at
    the registry gate and to within one bf16 ulp of its rounding."""
    b, inputs, outs, _ = run_registry("large_mm", seed=0)
    A, B = inputs
    got = outs[0]
    assert tuple(got.shape) == (8192, 8192)
    exact = oracle.matmul(oracle.as_f64(A), oracle.as_f64(B))
    assert_close(oracle.as_f64(got), exact, b.rtol, b.atol, "large_mm")
    _check_rounding(_bits(got).ravel(), exact.ravel(), "large_mm")


def test_kernel_attrs_report_register_split(mb):
    """mb_kernel_attrs_get reports the ArchVGPR / AGPR / SGPR counts of the
    kernel's own code object: each wave of the bf16 GEMM keeps its 128 x 128
    accumulator tile, 8 x 8 16x16 MFMA tiles of 4 fp32 per lane (256 per lane),
    in AGPRs, so one wave per SIMD fits."""
    a = native.kernel_attrs(native.kernel_find("large_matmul_bf16"))
    assert a["agprs"] == 256 and 0 < a["arch_vgprs"] <= 256, a
    assert a["arch_vgprs"] + a["agprs"] <= 512 and a["sgprs"] > 0
    assert a["waves_per_simd"] == 1 and a["static_lds_bytes"] == 163840
    for name in native.kernel_names():
        attrs = native.kernel_attrs(native.kernel_find(name))
        assert attrs["arch_vgprs"] > 0 and 1 <= attrs["waves_per_simd"] <= 8, (name, attrs)

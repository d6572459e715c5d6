"""fp32 MFMA GEMM (sqr_mm / rect_mm) on the GPU vs the float64 oracle.

Tolerance: rtol = atol = 1e-4 for the sqr_mm benchmark config, scaled with
sqrt(K) for the normal(0,1) shapes where |C| grows with K."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close, launch, ptr, run_registry, seeded

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n,k", [
    (1, 1, 1), (1, 64, 64), (64, 1, 64), (64, 64, 1), (64, 64, 64), (65, 33, 17),
    (128, 256, 64), (100, 300, 96), (257, 129, 200), (512, 512, 512), (31, 1000, 36),
    # fewer than 128 64x64 tiles and K <= 512 take the small-problem kernel
    # (32x32 tiles, K over up to 16 waves): K = 32 (one wave), 464 (15 waves,
    # the last one's slice half past K), ragged M and N
    (32, 96, 32), (96, 64, 464), (70, 130, 256),
    # full tiles with K % 256 == 0 and K >= 512 (and, at K = 512, at least 128
    # tiles) take the LDS-DMA kernel: two loop trips, three trips
    (1024, 512, 512), (192, 128, 768),
])
def test_matmul_f32_shapes(mb, dev, m, n, k):
    a = seeded(m * 1000 + k, (m, k), ("uniform", -1.0, 1.0))
    b = seeded(n * 1000 + k + 1, (k, n), ("uniform", -1.0, 1.0))
    d_a, d_b = a.to(dev), b.to(dev)
    d_c = torch.full((m, n), float("nan"), device=dev)
    launch("mb_launch_matmul_f32", ptr(d_a), ptr(d_b), ptr(d_c), m, n, k, None)
    want = oracle.matmul(a.numpy(), b.numpy())
    assert_close(d_c.cpu().numpy(), want, 1e-4, 1e-4, f"matmul_f32 {m}x{n}x{k}")


def _random_f32_shapes(n, seed=72):
    """Seeded shapes: half ragged, half full 64 x 64 tiles with K a multiple of
    256 from 512 (the LDS-DMA kernel from K = 768, the small-problem kernel at
    K = 512 when there are fewer than 128 tiles)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        if i % 2:
            out.append((64 * int(rng.integers(1, 9)), 64 * int(rng.integers(1, 9)),
                        256 * int(rng.integers(2, 5))))
        else:
            out.append(tuple(int(v) for v in rng.integers(1, 600, size=3)))
    return out


@pytest.mark.parametrize("m,n,k", _random_f32_shapes(8))
def test_matmul_f32_random_shapes(mb, dev, m, n, k):
    test_matmul_f32_shapes(mb, dev, m, n, k)


def test_matmul_f32_k0_gives_zeros(mb, dev):
    d_c = torch.full((8, 8), 5.0, device=dev)
    d_a = torch.zeros(1, device=dev)
    launch("mb_launch_matmul_f32", ptr(d_a), ptr(d_a), ptr(d_c), 8, 8, 0, None)
    assert torch.all(d_c.cpu() == 0.0)


# small-problem kernel, register-staged kernel (ragged), LDS-DMA kernel
@pytest.mark.parametrize("n", [192, 1000, 1024])
def test_matmul_f32_identity_exact(mb, dev, n):
    a = seeded(3, (n, n))
    eye = torch.eye(n)
    d_a, d_eye = a.to(dev), eye.to(dev)     # keep both alive across the launch
    d_c = torch.zeros((n, n), device=dev)
    launch("mb_launch_matmul_f32", ptr(d_a), ptr(d_eye), ptr(d_c), n, n, n, None)
    assert torch.equal(d_c.cpu(), a)


@pytest.mark.parametrize("name", ["sqr_mm", "rect_mm"])
def test_matmul_registry_config(mb, name):
    b, inputs, outs, _ = run_registry(name, seed=0)
    want = oracle.matmul(inputs[0].numpy(), inputs[1].numpy())
    tol = 1e-4 if name == "sqr_mm" else 1e-3
    assert_close(outs[0].numpy(), want, tol, tol, name)

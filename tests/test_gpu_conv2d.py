"""conv2d implicit GEMM (fp32 MFMA) on the GPU vs the float64 oracle.

Gate: rtol 1e-3 (benchmark configuration) with the registry's atol 1e-3."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close, launch, ptr, run_registry, seeded

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,h,w,c,o,r,s,st,pad", [
    (1, 8, 8, 32, 64, 3, 3, 1, 1),       # fast path, one tile
    (2, 9, 7, 64, 64, 3, 3, 1, 1),       # ragged M, borders
    (2, 10, 10, 64, 128, 3, 3, 1, 0),    # valid conv, two N tiles
    (1, 11, 13, 32, 40, 3, 3, 2, 1),     # stride 2, O not a tile multiple
    (3, 6, 6, 64, 64, 1, 1, 1, 0),       # 1x1 = GEMM
    (1, 7, 9, 3, 5, 3, 3, 1, 1),         # generic path (C % 32 != 0)
    (2, 5, 6, 20, 70, 2, 3, 1, 2),       # generic path, pad > filter/2
    (1, 3, 3, 32, 64, 5, 5, 1, 2),       # filter larger than the image interior
])
def test_conv2d_shapes(mb, dev, n, h, w, c, o, r, s, st, pad):
    x = seeded(n * h + c, (n, h, w, c))
    wt = seeded(o * r + s, (o, r, s, c), ("kaiming_normal", r * s * c))
    p = (h + 2 * pad - r) // st + 1
    q = (w + 2 * pad - s) // st + 1
    d_x, d_w = x.to(dev), wt.to(dev)
    d_y = torch.full((n, p, q, o), float("nan"), device=dev)
    launch("mb_launch_conv2d_nhwc_f32", ptr(d_x), ptr(d_w), ptr(d_y), n, h, w, c, o, r, s, st, pad,
           None)
    want = oracle.conv2d_nhwc(x.numpy(), wt.numpy(), st, pad)
    assert_close(d_y.cpu().numpy(), want, 1e-3, 1e-3, f"conv2d {n,h,w,c,o,r,s,st,pad}")


def _random_conv_shapes(n, seed=73):
    """Seeded geometries: channel counts of the fast path (multiples of 32) and
    of the generic one, 1x1 to 5x5 filters, stride 1 or 2, padding 0..2."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        r, s_ = int(rng.choice([1, 3, 5])), int(rng.choice([1, 3, 5]))
        st, pad = int(rng.choice([1, 2])), int(rng.integers(0, 3))
        nb, h, w = int(rng.integers(1, 4)), int(rng.integers(1, 17)), int(rng.integers(1, 17))
        c = int(rng.choice([32, 64, 96, 5, 20]))
        o = int(rng.integers(1, 140))
        if h + 2 * pad < r or w + 2 * pad < s_:
            continue
        out.append((nb, h, w, c, o, r, s_, st, pad))
    return out


@pytest.mark.parametrize("n,h,w,c,o,r,s,st,pad", _random_conv_shapes(10))
def test_conv2d_random_shapes(mb, dev, n, h, w, c, o, r, s, st, pad):
    test_conv2d_shapes(mb, dev, n, h, w, c, o, r, s, st, pad)


def test_conv2d_rejects_bad_geometry(mb, dev):
    from metalbench_amd import native
    lib = native.load()
    d = torch.zeros(16, device=dev)
    assert lib.mb_launch_conv2d_nhwc_f32(ptr(d), ptr(d), ptr(d), 1, 2, 2, 1, 1, 5, 5, 1, 0,
                                         None) == -7
    assert lib.mb_launch_conv2d_nhwc_f32(ptr(d), ptr(d), ptr(d), 1, 2, 2, 1, 1, 1, 1, 0, 0,
                                         None) == -7


@pytest.mark.parametrize("name", ["conv2d", "conv2d_ref"])
def test_conv2d_registry_config(mb, name):
    b, inputs, outs, _ = run_registry(name, seed=0)
    pad = b.meta["model_kwargs"]["padding"]
    want = oracle.conv2d_nhwc(inputs[0].numpy(), inputs[1].numpy(), 1, pad)
    assert_close(outs[0].numpy(), want, b.rtol, b.atol, name)

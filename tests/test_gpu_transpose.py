"""transpose_2d_f32 on the GPU vs the oracle: bit exact (reference registry
rtol = atol = 0, mlx/kernels/common/registry.py:165-179)."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import bits32, launch, ptr, run_bound, run_registry, seeded
from metalbench_amd import native

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols", [
    (1, 1), (1, 7), (7, 1), (64, 64), (63, 65), (65, 63), (128, 192), (1000, 3),
    (3, 1000), (333, 777), (1024, 2048), (2048, 1024), (4096, 64), (128, 128), (256, 384),
    (258, 386), (130, 4096),
])
def test_transpose_bit_exact(mb, dev, rows, cols):
    a = seeded(rows * 7919 + cols, (rows, cols))
    d_a = a.to(dev)
    d_b = torch.full((cols, rows), float("nan"), device=dev)
    launch("mb_launch_transpose_2d_f32", ptr(d_a), ptr(d_b), rows, cols, None)
    want = oracle.transpose(a.numpy())
    assert np.array_equal(bits32(d_b), want.view(np.int32))


@pytest.mark.parametrize("rows,cols", [tuple(int(v) for v in np.random.default_rng(74 + i)
                                                 .integers(1, 2500, size=2)) for i in range(8)])
def test_transpose_random_shapes_bit_exact(mb, dev, rows, cols):
    test_transpose_bit_exact(mb, dev, rows, cols)


def test_transpose_empty_is_noop(mb, dev):
    d_b = torch.full((4,), 3.0, device=dev)
    launch("mb_launch_transpose_2d_f32", ptr(d_b), ptr(d_b), 0, 4, None)
    assert torch.all(d_b.cpu() == 3.0)


def test_transpose_specials_bit_exact(mb, dev):
    # NaN payloads, infinities, signed zeros and denormals move unchanged.
    vals = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-45, -1e-40, 3.0],
                    np.float32)
    # 256 x 160: full 128 x 128 tiles (vector path) and an edge strip.
    a = np.resize(vals, (256, 160)).astype(np.float32)
    a.view(np.uint32)[5, 7] = 0x7FA00001            # signalling-NaN payload
    a.view(np.uint32)[200, 140] = 0xFFC00123
    d_a = torch.from_numpy(a).to(dev)
    d_b = torch.zeros((160, 256), device=dev)
    launch("mb_launch_transpose_2d_f32", ptr(d_a), ptr(d_b), 256, 160, None)
    assert np.array_equal(bits32(d_b), oracle.transpose(a).view(np.int32))


def test_transpose_unaligned_pointers_take_the_scalar_path(mb, dev):
    # A and B one float past a 16-byte boundary: full tiles, but no float4 access.
    rows, cols = 256, 384
    a = seeded(11, (rows, cols))
    buf_a = torch.zeros(rows * cols + 4, device=dev)
    buf_b = torch.full((rows * cols + 4,), float("nan"), device=dev)
    buf_a[1:1 + rows * cols] = a.reshape(-1).to(dev)
    launch("mb_launch_transpose_2d_f32", ptr(buf_a) + 4, ptr(buf_b) + 4, rows, cols, None)
    got = buf_b[1:1 + rows * cols].cpu().numpy().view(np.int32).reshape(cols, rows)
    assert np.array_equal(got, oracle.transpose(a.numpy()).view(np.int32))


@pytest.mark.parametrize("name", ["transpose_2d", "transpose_2d_ref"])
def test_transpose_registry_config(mb, name):
    b, inputs, outs, _ = run_registry(name, seed=0)
    want = oracle.transpose(inputs[0].numpy())
    assert np.array_equal(outs[0].numpy().view(np.int32), want.view(np.int32))


def test_cold_start_timing_evicts_and_keeps_results(mb):
    """mb_run with MB_RUN_COLD (the harness's --cold-start): every timed
    dispatch follows a cache eviction outside its event pair; the output is
    still bit exact, and the flag is refused with MB_RUN_WALL_ONLY."""
    import torch
    from metalbench_amd import helpers as H
    b = H.load_baseline("transpose_2d_ref")
    a = b.make_inputs(0)[0]
    (got,) = run_bound("transpose_2d_f32", [(0, a)], [(1, (2048, 1024))],
                       [(2, "u32", 1024), (3, "u32", 2048)])
    assert np.array_equal(bits32(got), bits32(a.t().contiguous()))
    dev = torch.device("cuda", 0)
    da, db = a.to(dev), torch.empty(2048, 1024, device=dev)
    binds = [native.make_binding(0, native.ROLE_INPUT, "f32", da.data_ptr(), da.numel() * 4),
             native.make_binding(1, native.ROLE_OUTPUT, "f32", db.data_ptr(), db.numel() * 4),
             native.make_binding(2, native.ROLE_SCALAR, "u32", value=1024),
             native.make_binding(3, native.ROLE_SCALAR, "u32", value=2048)]
    kid = native.kernel_find("transpose_2d_f32")
    t = native.run(kid, binds, 0, 3, native.RUN_COLD)
    assert t["iters"] == 3 and 0 < t["min_ms"] <= t["median_ms"]
    torch.cuda.synchronize()
    assert np.array_equal(bits32(db), bits32(a.t().contiguous()))
    with pytest.raises(native.NativeError) as e:
        native.run(kid, binds, 0, 2, native.RUN_COLD | native.RUN_WALL_ONLY)
    assert e.value.code == -7


@pytest.mark.parametrize("n", [1, 3, 4, 1023, 4096, 4096 * 257 + 5])
def test_copy_bit_exact(mb, dev, n):
    """The copy kernel (the HBM-ceiling and counter-calibration kernel that
    bench.py runs): bit-exact for any length, the tail past the last whole
    16-byte vector included."""
    a = seeded(n, (n,))
    d_a = a.to(dev)
    d_b = torch.full((n,), float("nan"), device=dev)
    launch("mb_launch_copy_f32", ptr(d_a), ptr(d_b), n, None)
    assert np.array_equal(bits32(d_b), a.numpy().view(np.int32))


@pytest.mark.parametrize("n", [1, 5, 4096 * 257 + 3])
def test_plain_copy_bit_exact(mb, dev, n):
    """copy_f32_plain (cached accesses: the FETCH_SIZE / WRITE_SIZE
    calibration kernel) through mb_run: bit-exact, tail included."""
    a = seeded(n + 7, (n,))
    d_a = a.to(dev)
    d_b = torch.full((n,), float("nan"), device=dev)
    binds = [native.make_binding(0, native.ROLE_INPUT, "f32", ptr(d_a), 4 * n),
             native.make_binding(1, native.ROLE_OUTPUT, "f32", ptr(d_b), 4 * n),
             native.make_binding(2, native.ROLE_SCALAR, "u32", value=n)]
    native.run(native.kernel_find("copy_f32_plain"), binds, 0, 1, native.RUN_SYNC_EACH)
    torch.cuda.synchronize()
    assert np.array_equal(bits32(d_b), a.numpy().view(np.int32))

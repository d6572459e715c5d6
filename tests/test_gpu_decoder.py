"""LLaMA decoder decode step on the GPU vs the float64 oracle.

Gate (benchmark configuration): rtol 2e-2 with atol 2e-2 (outputs are O(1)), on y, k_new and
v_new.  Covers batch 1..16, empty / short / chunk-boundary caches, GQA group
sizes 1..16, padded cache strides, tensor-parallel shards, shapes whose QKV
tiles take class-dependent K splits, a seeded sweep of random shapes, the
caller-workspace path, repeat calls (self-resetting split-K counters must give
bit-identical results) and the full registry configuration."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close, run_registry, seeded
from metalbench_amd import native

pytestmark = pytest.mark.gpu

RTOL = ATOL = 2e-2


def _make(B, D, H, HKV, FF, L, stride=None, seed=0):
    dh = 128
    qd = H * dh   # the attention width: D for a whole layer, less for one shard
    stride = stride or L
    s = seed * 100
    bf = "bf16"
    ins = dict(
        x=seeded(s + 1, (B, D), ("normal", 0.0, 1.0), bf),
        w_qkv=seeded(s + 2, (D, qd + 2 * HKV * dh), ("normal", 0.0, 0.02), bf),
        w_o=seeded(s + 3, (qd, D), ("normal", 0.0, 0.02), bf),
        w_gu=seeded(s + 4, (D, 2 * FF), ("normal", 0.0, 0.02), bf),
        w_down=seeded(s + 5, (FF, D), ("normal", 0.0, 0.02), bf),
        k_cache=seeded(s + 6, (B, HKV, stride, dh), ("normal", 0.0, 1.0), bf),
        v_cache=seeded(s + 7, (B, HKV, stride, dh), ("normal", 0.0, 1.0), bf),
    )
    return ins


def _run(dev, ins, B, D, H, HKV, FF, L, stride=None, workspace=None):
    stride = stride or L
    d = {k: v.to(dev) for k, v in ins.items()}
    y = torch.full((B, D), float("nan"), dtype=torch.bfloat16, device=dev)
    kn = torch.full((B, HKV, 128), float("nan"), dtype=torch.bfloat16, device=dev)
    vn = torch.full((B, HKV, 128), float("nan"), dtype=torch.bfloat16, device=dev)
    a = native.MbDecoderStepArgs(
        batch=B, d_model=D, n_heads=H, n_kv_heads=HKV, head_dim=128, d_ff=FF, cache_len=L,
        cache_stride=stride, rope_base=500000.0, eps=1e-5,
        x=d["x"].data_ptr(), w_qkv=d["w_qkv"].data_ptr(), w_o=d["w_o"].data_ptr(),
        w_gu=d["w_gu"].data_ptr(), w_down=d["w_down"].data_ptr(),
        k_cache=d["k_cache"].data_ptr(), v_cache=d["v_cache"].data_ptr(),
        y=y.data_ptr(), k_new=kn.data_ptr(), v_new=vn.data_ptr(),
        workspace=workspace.data_ptr() if workspace is not None else None,
        workspace_bytes=workspace.numel() if workspace is not None else 0)
    torch.cuda.synchronize()
    native.check("mb_launch_llama_decoder_step_bf16",
                 native.load().mb_launch_llama_decoder_step_bf16(ctypes.byref(a), None))
    torch.cuda.synchronize()
    return y.cpu(), kn.cpu(), vn.cpu()


def _want(ins, H, HKV, L):
    f = oracle.as_f64
    kc = f(ins["k_cache"])[:, :, :L]
    vc = f(ins["v_cache"])[:, :, :L]
    return oracle.llama_decoder_step(f(ins["x"]), f(ins["w_qkv"]), f(ins["w_o"]), f(ins["w_gu"]),
                                     f(ins["w_down"]), kc, vc, n_heads=H, n_kv_heads=HKV,
                                     head_dim=128)


def _check(got, want, what):
    for g, w, name in zip(got, want, ("y", "k_new", "v_new")):
        assert_close(oracle.as_f64(g), w, RTOL, ATOL, f"{what} {name}")


@pytest.mark.parametrize("B,D,H,HKV,FF,L", [
    (2, 512, 4, 2, 1024, 40),      # smoke shape
    (1, 256, 2, 1, 384, 0),        # empty cache: attends to itself only; 128-col gate|up tiles
    (2, 512, 4, 2, 512, 0),        # empty cache
    (3, 512, 4, 4, 256, 5),        # MHA (G = 1)
    (4, 512, 4, 4, 512, 5),        # MHA (G = 1)
    (16, 1024, 8, 1, 512, 128),    # G = 8, one full 128-key split + the new key
    (5, 512, 4, 2, 640, 129),      # split boundary + 1
    (7, 1024, 8, 2, 1024, 300),    # several 64-key blocks, ragged
    (16, 2048, 16, 4, 1536, 1000),  # GQA 4 as the full config, several splits
    (9, 2048, 16, 1, 1024, 77),    # G = 16
    (4, 4096, 16, 4, 2048, 64),    # QKV tiles of the slow address class take 11 K splits, others 10
])
def test_decoder_step_shapes(mb, dev, B, D, H, HKV, FF, L):
    ins = _make(B, D, H, HKV, FF, L)
    _check(_run(dev, ins, B, D, H, HKV, FF, L), _want(ins, H, HKV, L), f"{B,D,H,HKV,FF,L}")


@pytest.mark.parametrize("B,D,H,HKV,FF,L", [
    (16, 4096, 4, 1, 1792, 2048),  # one GPU's share of the registry step at 8-way TP
    (16, 4096, 8, 2, 3584, 300),   # a 4-way share, ragged cache
    (3, 1024, 1, 1, 256, 65),      # one head of a layer with D = 1024
    (2, 8192, 1, 1, 256, 64),      # 32 QKV K splits: the attention prologue sums two batches
    (1, 16384, 1, 1, 128, 16),     # 64 QKV K splits, the widest d_model
])
def test_decoder_step_tensor_parallel_shard(mb, dev, B, D, H, HKV, FF, L):
    """One tensor-parallel shard (attention width H * 128 < D): the shard's
    QKV columns, W_o rows and FFN slice, all-reduces left to the caller."""
    ins = _make(B, D, H, HKV, FF, L)
    _check(_run(dev, ins, B, D, H, HKV, FF, L), _want(ins, H, HKV, L), f"shard {B,D,H,HKV,FF,L}")


def _random_shapes(n, seed=20261202):
    """Seeded decode-step shapes inside the kernel's limits: batch 1..16,
    d_model a multiple of 128, query heads a multiple of kv heads (G <= 16,
    the attention width below or equal to d_model), d_ff a multiple of 128,
    cache 0..700 keys with an optional padded stride."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        B = int(rng.integers(1, 17))
        D = 128 * int(rng.integers(2, 25))            # 256 .. 3072
        HKV = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.choice([1, 2, 4, 8, 16]))
        H = HKV * G
        if H * 128 > D:
            continue
        FF = 128 * int(rng.integers(1, 25))           # 128 .. 3072
        L = int(rng.integers(0, 701))
        S = L + int(rng.choice([0, 0, 1, 37]))
        out.append((B, D, H, HKV, FF, L, S))
    return out


@pytest.mark.parametrize("B,D,H,HKV,FF,L,S", _random_shapes(10))
def test_decoder_step_random_shapes(mb, dev, B, D, H, HKV, FF, L, S):
    """A seeded sweep over the plan's shape space (split counts, ring depth,
    attention splits, shard widths, strides) against the oracle."""
    ins = _make(B, D, H, HKV, FF, L, stride=max(S, 1), seed=B + D + L)
    _check(_run(dev, ins, B, D, H, HKV, FF, L, stride=max(S, 1)), _want(ins, H, HKV, L),
           f"random {B,D,H,HKV,FF,L,S}")


def test_decoder_step_new_inputs_every_call(mb, dev):
    """Back-to-back steps on different data through one workspace: no call may
    see an earlier call's intermediates (queries, attention, x1, SwiGLU)."""
    cfg = (16, 1024, 8, 2, 1024, 256)
    B, D, H, HKV, FF, L = cfg
    for seed in (21, 22, 23):
        ins = _make(*cfg, seed=seed)
        _check(_run(dev, ins, *cfg), _want(ins, H, HKV, L), f"seed {seed}")


def test_decoder_step_padded_stride_and_caller_workspace(mb, dev):
    B, D, H, HKV, FF, L, S = 4, 512, 4, 2, 512, 70, 96
    ins = _make(B, D, H, HKV, FF, L, stride=S, seed=3)
    a = native.MbDecoderStepArgs(batch=B, d_model=D, n_heads=H, n_kv_heads=HKV, head_dim=128,
                                 d_ff=FF, cache_len=L, cache_stride=S, rope_base=500000.0,
                                 eps=1e-5)
    nbytes = native.load().mb_decoder_step_workspace_bytes(ctypes.byref(a))
    assert nbytes > 0
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    got_ws = _run(dev, ins, B, D, H, HKV, FF, L, stride=S, workspace=ws)
    got_lib = _run(dev, ins, B, D, H, HKV, FF, L, stride=S)
    _check(got_ws, _want(ins, H, HKV, L), "caller workspace")
    for g1, g2 in zip(got_ws, got_lib):
        assert torch.equal(g1, g2)
    # the caller's workspace is left ready: a second call gives the same bits
    for g1, g2 in zip(got_ws, _run(dev, ins, B, D, H, HKV, FF, L, stride=S, workspace=ws)):
        assert torch.equal(g1, g2)
    # and it needs no initialisation: a workspace of 0xff bytes (every counter
    # far from zero) gives the same bits too
    junk = torch.full((nbytes,), 255, dtype=torch.uint8, device=dev)
    for g1, g2 in zip(got_ws, _run(dev, ins, B, D, H, HKV, FF, L, stride=S, workspace=junk)):
        assert torch.equal(g1, g2)


def test_decoder_step_repeat_calls_bit_identical(mb, dev):
    B, D, H, HKV, FF, L = 16, 1024, 8, 2, 1024, 256
    ins = _make(B, D, H, HKV, FF, L, seed=5)
    first = _run(dev, ins, B, D, H, HKV, FF, L)
    for _ in range(3):
        again = _run(dev, ins, B, D, H, HKV, FF, L)
        for g1, g2 in zip(first, again):
            assert torch.equal(g1, g2)


def test_decoder_step_rejects_bad_shapes(mb, dev):
    lib = native.load()
    a = native.MbDecoderStepArgs(batch=17, d_model=512, n_heads=4, n_kv_heads=2, head_dim=128,
                                 d_ff=512, cache_len=4, cache_stride=4, rope_base=5e5, eps=1e-5)
    assert lib.mb_launch_llama_decoder_step_bf16(ctypes.byref(a), None) == -7
    a.batch, a.n_kv_heads = 4, 3
    assert lib.mb_launch_llama_decoder_step_bf16(ctypes.byref(a), None) == -7
    a.n_kv_heads, a.cache_stride = 2, 2
    assert lib.mb_launch_llama_decoder_step_bf16(ctypes.byref(a), None) == -7
    a.cache_stride, a.d_model = 4, 500          # residual width not a multiple of 128
    assert lib.mb_launch_llama_decoder_step_bf16(ctypes.byref(a), None) == -7


def test_decoder_step_registry_config(mb):
    """Full benchmark config: B 16, D 4096, 32/8 heads, FF 14336, L 2048."""
    b, inputs, outs, k_t = run_registry("llama_decoder_step", seed=0, warmup=1, iters=3)
    f = oracle.as_f64
    want = oracle.llama_decoder_step(*[f(t) for t in inputs], n_heads=32, n_kv_heads=8)
    for got, w, name in zip(outs, want, ("y", "k_new", "v_new")):
        assert_close(f(got), w, RTOL, ATOL, f"llama_decoder_step {name}")


def test_decoder_step_library_workspace_across_shape_changes(mb, dev):
    """Counters sit at the front of the shared library workspace; a call with
    fewer counters writes scratch data past them, so a following call with
    more counters must clear them first (regression test)."""
    big = (16, 2048, 16, 4, 1536, 1000)
    small = (4, 512, 4, 2, 512, 70)
    mid = (16, 1024, 8, 2, 1024, 256)
    for cfg in (big, small, mid, small, big):
        ins = _make(*cfg, seed=7)
        B, D, H, HKV, FF, L = cfg
        _check(_run(dev, ins, *cfg), _want(ins, H, HKV, L), f"sequence {cfg}")


def test_decoder_workspace_size_does_not_depend_on_init(dev):
    """mb_decoder_step_workspace_bytes() is callable before mb_init() and must
    give the size a launch after mb_init() checks against."""
    cfg = (16, 2048, 16, 4, 1536, 1000)
    B, D, H, HKV, FF, L = cfg
    a = native.MbDecoderStepArgs(batch=B, d_model=D, n_heads=H, n_kv_heads=HKV, head_dim=128,
                                 d_ff=FF, cache_len=L, cache_stride=L, rope_base=500000.0,
                                 eps=1e-5)
    native.shutdown()
    before = native.load().mb_decoder_step_workspace_bytes(ctypes.byref(a))
    native.init(0)
    after = native.load().mb_decoder_step_workspace_bytes(ctypes.byref(a))
    assert before == after > 0
    ins = _make(*cfg, seed=11)
    ws = torch.zeros(before, dtype=torch.uint8, device=dev)
    _check(_run(dev, ins, *cfg, workspace=ws), _want(ins, H, HKV, L), "pre-init workspace size")


def test_decoder_step_rope_at_large_position(mb, dev):
    """The new token at position 10^6: its RoPE angle pos * base^(-2i/Dh) must be
    formed in fp64 (in fp32 the first pairs' angles are off by 0.03-0.08 rad,
    i.e. several percent of k_new, far above bf16 rounding)."""
    B, D, H, HKV, FF, L = 1, 256, 2, 1, 256, 1_000_000
    ins = _make(B, D, H, HKV, FF, L, seed=13)
    got = _run(dev, ins, B, D, H, HKV, FF, L)
    want = _want(ins, H, HKV, L)
    _check(got, want, "pos 1e6")
    kn, wk = oracle.as_f64(got[1]), want[1]
    pair = np.sqrt(wk[..., 0::2] ** 2 + wk[..., 1::2] ** 2).repeat(2, axis=-1)
    bad = np.abs(kn - wk) > 2.0 ** -8 * np.abs(wk) + 1e-4 * pair
    assert not bad.any(), f"k_new: {int(bad.sum())} of {kn.size} beyond bf16 rounding, " \
                          f"max |diff| {np.abs(kn - wk).max():.3e}"


def test_decoder_parts_time_each_kernel_alone(mb):
    """mb_run with MB_RUN_PARTS: the decode step reports its five kernels by
    name, each timed by its own start and end events (hipExtLaunchKernel), so
    every part is positive and the parts sum to less than the whole dispatch,
    which also holds the dispatch gaps between them.  The outputs of a timed
    run are the step's (checked against the oracle at the registry shape by
    test_decoder_step_registry_config)."""
    from metalbench_amd import harness
    from metalbench_amd import helpers as H
    b = H.load_baseline("llama_decoder_step_tp8")
    k_t, outs = harness._run_native(b, b.make_inputs(0), 1, 5,
                                    native.RUN_PIPELINED | native.RUN_PARTS)
    names = [p["name"] for p in k_t["parts"]]
    assert names == ["qkv", "attention", "wo_residual", "gate_up_swiglu", "down_residual"]
    assert all(p["mean_ms"] > 0 for p in k_t["parts"]), k_t["parts"]
    assert sum(p["mean_ms"] for p in k_t["parts"]) < k_t["mean_ms"], k_t
    assert all(torch.isfinite(o.float()).all() for o in outs)

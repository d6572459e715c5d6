"""The allocation-free decoder entry point against the allocating one.

mb_launch_llama_decoder_step_bf16_noalloc runs the same kernels on a static
device scratch; it must give bit-identical y, k_new and v_new to
mb_launch_llama_decoder_step_bf16 (the decoder's own parity tests tie that
entry point to the float64 oracle), on two calls in a row with the second one
smaller, replay from a captured HIP graph, and reject shapes beyond its
scratch size without touching the GPU."""
import ctypes

import pytest
import torch

from gpu_util import seeded
from metalbench_amd import native

pytestmark = pytest.mark.gpu


def _args(dev, cfg, seed):
    B, D, H, HKV, FF, L = cfg
    dh = 128
    bf = "bf16"
    s = 1000 + seed * 10
    ins = [seeded(s + 1, (B, D), ("normal", 0.0, 1.0), bf),
           seeded(s + 2, (D, D + 2 * HKV * dh), ("normal", 0.0, 0.02), bf),
           seeded(s + 3, (D, D), ("normal", 0.0, 0.02), bf),
           seeded(s + 4, (D, 2 * FF), ("normal", 0.0, 0.02), bf),
           seeded(s + 5, (FF, D), ("normal", 0.0, 0.02), bf),
           seeded(s + 6, (B, HKV, L, dh), ("normal", 0.0, 1.0), bf),
           seeded(s + 7, (B, HKV, L, dh), ("normal", 0.0, 1.0), bf)]
    d = [t.to(dev) for t in ins]
    outs = [torch.full(shape, float("nan"), dtype=torch.bfloat16, device=dev)
            for shape in ((B, D), (B, HKV, dh), (B, HKV, dh))]
    a = native.MbDecoderStepArgs(
        batch=B, d_model=D, n_heads=H, n_kv_heads=HKV, head_dim=dh, d_ff=FF, cache_len=L,
        cache_stride=L, rope_base=500000.0, eps=1e-5,
        x=d[0].data_ptr(), w_qkv=d[1].data_ptr(), w_o=d[2].data_ptr(), w_gu=d[3].data_ptr(),
        w_down=d[4].data_ptr(), k_cache=d[5].data_ptr(), v_cache=d[6].data_ptr(),
        y=outs[0].data_ptr(), k_new=outs[1].data_ptr(), v_new=outs[2].data_ptr(),
        workspace=None, workspace_bytes=0)
    return a, d, outs


def _call(fn, a):
    torch.cuda.synchronize()
    native.check(fn, getattr(native.load(), fn)(ctypes.byref(a), None))
    torch.cuda.synchronize()


def test_noalloc_matches_allocating_entry_point(mb, dev):
    print("[no-alloc] two calls, the second smaller", flush=True)
    for seed, cfg in enumerate(((16, 2048, 16, 4, 1536, 1000), (4, 512, 4, 2, 512, 70))):
        a, d, outs = _args(dev, cfg, seed)
        _call("mb_launch_llama_decoder_step_bf16_noalloc", a)
        got = [t.clone() for t in outs]
        for t in outs:
            t.fill_(float("nan"))
        _call("mb_launch_llama_decoder_step_bf16", a)
        for g, w, name in zip(got, outs, ("y", "k_new", "v_new")):
            assert not torch.isnan(g.float()).any(), f"{cfg} {name}: not written"
            assert torch.equal(g, w), f"{cfg} {name}: no-alloc result differs"


def test_noalloc_step_replays_from_captured_graphs(mb, dev):
    """The entry point's purpose: callers that capture the step in HIP graphs
    (one per shape, as serving loops do).  Two shapes are captured after one
    eager call each; the graphs are then replayed three times each,
    interleaved with eager calls of a smaller third shape on the same
    scratch, with synchronisation between; every replay must reproduce the
    eager outputs bit for bit."""
    print("[no-alloc] graph capture and interleaved replays", flush=True)
    lib = native.load()
    fn = lib.mb_launch_llama_decoder_step_bf16_noalloc
    cases = []
    for seed, cfg in ((7, (4, 512, 4, 2, 512, 70)), (8, (16, 2048, 16, 4, 1536, 300))):
        a, d, outs = _args(dev, cfg, seed)
        _call("mb_launch_llama_decoder_step_bf16_noalloc", a)
        want = [t.clone() for t in outs]
        stream = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            rc = fn(ctypes.byref(a), ctypes.c_void_p(stream.cuda_stream))
        assert rc == 0, native.last_error()
        cases.append((cfg, graph, outs, want, a, d))
    a3, d3, outs3 = _args(dev, (2, 256, 2, 1, 256, 10), 9)
    for rep in range(3):
        for cfg, graph, outs, want, _, _ in reversed(cases):
            _call("mb_launch_llama_decoder_step_bf16_noalloc", a3)   # other shapes in between
            for t in outs:
                t.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for g, w, name in zip(outs, want, ("y", "k_new", "v_new")):
                assert torch.equal(g, w), f"replay {rep} {cfg} {name}: differs from the eager call"


def test_noalloc_rejects_oversized_shapes_and_a_workspace(mb, dev):
    lib = native.load()
    # d_ff 14336 * 16: the SwiGLU activations and split-K partials need 43 MiB
    a = native.MbDecoderStepArgs(batch=16, d_model=4096, n_heads=32, n_kv_heads=8, head_dim=128,
                                 d_ff=14336 * 16, cache_len=16, cache_stride=16,
                                 rope_base=500000.0, eps=1e-5)
    need = lib.mb_decoder_step_workspace_bytes(ctypes.byref(a))
    assert need > (32 << 20)
    assert lib.mb_launch_llama_decoder_step_bf16_noalloc(ctypes.byref(a), None) == -7
    assert "static scratch holds" in native.last_error()
    a2, d, outs = _args(dev, (4, 512, 4, 2, 512, 70), 5)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    a2.workspace, a2.workspace_bytes = ws.data_ptr(), ws.numel()
    assert lib.mb_launch_llama_decoder_step_bf16_noalloc(ctypes.byref(a2), None) == -7
    assert "workspace must be NULL" in native.last_error()

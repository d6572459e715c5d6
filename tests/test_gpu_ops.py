"""Decoder sub-ops and adjacent GEMMs on the GPU vs the float64 oracle.

Each registry entry runs at the reference's own shape and tolerance (the
registry's rtol/atol), then at ragged shapes that take the kernels' scalar
and multi-block paths.  Inputs are seeded normal(0, 1), like the reference's;
for the attention blocks at ragged shapes the weights are scaled by 1/sqrt(D)
so that the softmax is not one-hot (a near-tie between two keys would then
decide the output)."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close, run_bound, run_registry, seeded

pytestmark = pytest.mark.gpu

f64 = oracle.as_f64


def _registry_check(name, want_fn):
    b, inputs, outs, _ = run_registry(name, seed=0, warmup=1, iters=2)
    want = want_fn(*[f64(t) for t in inputs])
    assert_close(f64(outs[0]), want, b.rtol, b.atol, name)


def test_rms_norm_registry():
    _registry_check("rms_norm", lambda x: oracle.rms_norm(x, 1e-5))


def test_fused_add_rms_norm_registry():
    _registry_check("fused_add_rms_norm", lambda x, r: oracle.fused_add_rms_norm(x, r, 1e-5))


def test_rms_norm_linear_registry():
    _registry_check("rms_norm_linear", lambda x, w: oracle.rms_norm_linear(x, w, 1e-5))


def test_rope_embedding_registry():
    _registry_check("rope_embedding", lambda x: oracle.rope_embedding(x, 10000.0))


def test_swiglu_registry():
    _registry_check("swiglu", oracle.swiglu)


def test_fused_qkv_projection_registry():
    _registry_check("fused_qkv_projection", oracle.matmul)


def test_matvec_registry():
    _registry_check("matvec", oracle.matmul)


def test_batch_mm_registry():
    _registry_check("batch_mm", oracle.matmul)


def test_llama_attention_registry():
    _registry_check("llama_attention", lambda x, wq, wo: oracle.llama_attention(
        x, wq, wo, n_heads=4, n_kv_heads=2, base=10000.0))


def test_llama_decoder_layer_registry():
    _registry_check("llama_decoder_layer", lambda x, wq, wo, wgu, wd: oracle.llama_decoder_layer(
        x, wq, wo, wgu, wd, n_heads=4, n_kv_heads=2, base=10000.0, eps=1e-5))


# ---- ragged shapes ------------------------------------------------------------------------

@pytest.mark.parametrize("rows,cols", [(7, 100), (33, 1000), (5, 4096), (1, 4)])
def test_rms_norm_shapes(mb, rows, cols):
    x = seeded(1, (rows, cols))
    (y,) = run_bound("rms_norm_f32", [(0, x)], [(1, (rows, cols))],
                     [(2, "u32", cols), (3, "f32", 1e-5)])
    assert_close(f64(y), oracle.rms_norm(f64(x), 1e-5), 1e-3, 1e-3, f"rms_norm {rows}x{cols}")


@pytest.mark.parametrize("rows,cols", [(33, 260), (3, 7)])
def test_fused_add_rms_norm_shapes(mb, rows, cols):
    x, r = seeded(2, (rows, cols)), seeded(3, (rows, cols))
    (y,) = run_bound("fused_add_rms_norm_f32", [(0, x), (1, r)], [(2, (rows, cols))],
                     [(3, "u32", cols), (4, "f32", 1e-5)])
    assert_close(f64(y), oracle.fused_add_rms_norm(f64(x), f64(r), 1e-5), 1e-3, 1e-3,
                 f"fused_add_rms_norm {rows}x{cols}")


@pytest.mark.parametrize("m,n,k", [(70, 90, 130), (64, 64, 64), (1, 3, 5),
                                   # full 64-tiles, K a multiple of 256: the LDS-DMA kernel
                                   (128, 192, 512), (64, 320, 768), (192, 64, 1024)])
def test_rms_norm_linear_shapes(mb, m, n, k):
    x, w = seeded(4, (m, k)), seeded(5, (n, k))
    (y,) = run_bound("rms_norm_linear_f32", [(0, x), (1, w)], [(2, (m, n))],
                     [(3, "u32", m), (4, "u32", n), (5, "u32", k), (6, "f32", 1e-5)])
    assert_close(f64(y), oracle.rms_norm_linear(f64(x), f64(w), 1e-5), 1e-3, 1e-3,
                 f"rms_norm_linear {m,n,k}")


@pytest.mark.parametrize("m,n,k", [(100, 70, 36), (65, 130, 257)])
def test_swiglu_shapes(mb, m, n, k):
    x, wg, wu = seeded(6, (m, k)), seeded(7, (k, n)), seeded(8, (k, n))
    (y,) = run_bound("swiglu_f32", [(0, x), (1, wg), (2, wu)], [(3, (m, n))],
                     [(4, "u32", m), (5, "u32", n), (6, "u32", k)])
    assert_close(f64(y), oracle.swiglu(f64(x), f64(wg), f64(wu)), 1e-3, 1e-3, f"swiglu {m,n,k}")


@pytest.mark.parametrize("batch,m,n,k", [(3, 70, 50, 33), (2, 64, 128, 256), (2, 64, 128, 512)])
def test_batch_mm_shapes(mb, batch, m, n, k):
    a, b = seeded(9, (batch, m, k)), seeded(10, (batch, k, n))
    (c,) = run_bound("batch_matmul_f32", [(0, a), (1, b)], [(2, (batch, m, n))],
                     [(3, "u32", m), (4, "u32", n), (5, "u32", k)])
    assert_close(f64(c), oracle.matmul(f64(a), f64(b)), 1e-3, 1e-3, f"batch_mm {batch,m,n,k}")


@pytest.mark.parametrize("m,k", [(77, 1001), (3, 4096), (5, 1)])
def test_matvec_shapes(mb, m, k):
    a, v = seeded(11, (m, k)), seeded(12, (k,))
    (y,) = run_bound("matvec_f32", [(0, a), (1, v)], [(2, (m,))], [(3, "u32", k)])
    assert_close(f64(y), oracle.matmul(f64(a), f64(v)), 1e-3, 1e-3, f"matvec {m,k}")


@pytest.mark.parametrize("s,d", [(5, 10), (300, 128), (1, 2)])
def test_rope_embedding_shapes(mb, s, d):
    x = seeded(13, (s, d))
    (y,) = run_bound("rope_embedding_f32", [(0, x)], [(1, (s, d))],
                     [(2, "u32", s), (3, "u32", d), (4, "f32", 10000.0)])
    assert_close(f64(y), oracle.rope_embedding(f64(x), 10000.0), 1e-4, 1e-5, f"rope {s}x{d}")


def _attn_inputs(s, d, h, hkv, seed):
    dh = d // h
    x = seeded(seed, (s, d))
    wq = seeded(seed + 1, (d, d + 2 * hkv * dh), ("normal", 0.0, d ** -0.5))
    wo = seeded(seed + 2, (d, d), ("normal", 0.0, d ** -0.5))
    return x, wq, wo


@pytest.mark.parametrize("s,d,h,hkv", [(70, 256, 4, 1), (1, 128, 4, 2), (130, 128, 1, 1),
                                       (64, 256, 8, 8)])
def test_llama_attention_shapes(mb, s, d, h, hkv):
    x, wq, wo = _attn_inputs(s, d, h, hkv, 20)
    (y,) = run_bound("llama_attention_f32", [(0, x), (1, wq), (2, wo)], [(3, (s, d))],
                     [(4, "u32", s), (5, "u32", d), (6, "u32", h), (7, "u32", hkv),
                      (8, "f32", 10000.0)])
    want = oracle.llama_attention(f64(x), f64(wq), f64(wo), n_heads=h, n_kv_heads=hkv)
    assert_close(f64(y), want, 1e-2, 1e-2, f"llama_attention {s,d,h,hkv}")


@pytest.mark.parametrize("s,d,h,hkv,ff", [(100, 256, 8, 2, 320), (1, 128, 4, 2, 256),
                                          (65, 128, 2, 1, 100)])
def test_llama_decoder_layer_shapes(mb, s, d, h, hkv, ff):
    x, wq, wo = _attn_inputs(s, d, h, hkv, 30)
    wgu = seeded(34, (d, 2 * ff), ("normal", 0.0, d ** -0.5))
    wd = seeded(35, (ff, d), ("normal", 0.0, ff ** -0.5))
    (y,) = run_bound("llama_decoder_layer_f32",
                     [(0, x), (1, wq), (2, wo), (3, wgu), (4, wd)], [(5, (s, d))],
                     [(6, "u32", s), (7, "u32", d), (8, "u32", h), (9, "u32", hkv),
                      (10, "u32", ff), (11, "f32", 10000.0), (12, "f32", 1e-5)])
    want = oracle.llama_decoder_layer(f64(x), f64(wq), f64(wo), f64(wgu), f64(wd), n_heads=h,
                                      n_kv_heads=hkv, base=10000.0, eps=1e-5)
    assert_close(f64(y), want, 1e-2, 1e-2, f"llama_decoder_layer {s,d,h,hkv,ff}")


def test_rejects_bad_shapes(mb):
    import ctypes  # noqa: F401
    from metalbench_amd import native
    x = seeded(40, (4, 96))
    with pytest.raises(native.NativeError):   # head dim 96 / 4 = 24: unsupported
        run_bound("llama_attention_f32", [(0, x), (1, seeded(41, (96, 96 + 2 * 24))),
                                          (2, seeded(42, (96, 96)))], [(3, (4, 96))],
                  [(4, "u32", 4), (5, "u32", 96), (6, "u32", 4), (7, "u32", 1),
                   (8, "f32", 10000.0)])
    with pytest.raises(native.NativeError):   # odd D
        run_bound("rope_embedding_f32", [(0, seeded(43, (3, 5)))], [(1, (3, 5))],
                  [(2, "u32", 3), (3, "u32", 5), (4, "f32", 10000.0)])

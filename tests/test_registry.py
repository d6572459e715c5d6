"""Registry entries, spec loading, seeded inputs and the Model specs (CPU)."""
import math

import numpy as np
import pytest
import torch

import oracle
from metalbench_amd import helpers as H

ALL = H.all_kernels()


@pytest.mark.parametrize("set_name", ["common", "full"])
def test_registry_nonempty_standalone_exec(set_name):
    # reference tests/metalbench/test_bench_smoke.py:27-34: registry.py exec'd on its own
    ns = {}
    exec((H.BASELINE_ROOT / set_name / "registry.py").read_text(), ns)
    assert ns.get("REGISTRY")


@pytest.mark.parametrize("set_name,name", ALL)
def test_entry_loads_and_validates(set_name, name):
    b = H.load_baseline(name)
    n_in = len(b.meta["input_shapes"])
    assert b.outputs[0].binding == n_in                      # reference mlx_helpers.py:259-263
    used = set(b.input_bindings) | {o.binding for o in b.outputs} | {s.binding for s in b.scalars()}
    assert len(used) == n_in + len(b.outputs) + len(b.scalars())   # no binding reused
    assert all(0 <= i < 32 for i in used)
    assert H.find_kernel_source(name) is not None, f"no HIP source registers {b.metal_function}"


def test_baseline_flops_and_bytes_match_baseline_md():
    m = {n: H.load_baseline(n).meta for n in ("sqr_mm", "transpose_2d", "conv2d", "large_mm",
                                               "llama_decoder_step")}
    assert (m["sqr_mm"]["flops"], m["sqr_mm"]["bytes"]) == (2_147_483_648, 12_582_912)
    assert (m["transpose_2d"]["flops"], m["transpose_2d"]["bytes"]) == (0, 536_870_912)
    assert (m["conv2d"]["flops"], m["conv2d"]["bytes"]) == (7_398_752_256, 51_527_680)
    assert (m["large_mm"]["flops"], m["large_mm"]["bytes"]) == (1_099_511_627_776, 402_653_184)
    assert (m["llama_decoder_step"]["flops"], m["llama_decoder_step"]["bytes"]) == \
        (7_516_454_912, 570_753_024)


def test_inputs_are_seeded_and_follow_their_distributions():
    b = H.load_baseline("sqr_mm")
    x1, x2 = b.make_inputs(0), b.make_inputs(0)
    assert all(torch.equal(a, c) for a, c in zip(x1, x2))
    assert not torch.equal(b.make_inputs(1)[0], x1[0])
    a = x1[0]
    assert a.dtype == torch.float32 and a.min() >= -1 and a.max() <= 1
    assert abs(a.mean().item()) < 0.01 and abs(a.std().item() - 1 / math.sqrt(3)) < 0.01

    gen = torch.Generator().manual_seed(0)
    w = H.generate_input(gen, (64, 3, 3, 64), ("kaiming_normal", 576))
    assert abs(w.std().item() - math.sqrt(2 / 576)) < 0.002
    t = H.generate_input(gen, (512, 512), ("normal", 0.0, 0.02), "bf16")
    assert t.dtype == torch.bfloat16 and abs(t.float().std().item() - 0.02) < 0.0005


def test_bad_registry_entries_are_rejected():
    with pytest.raises(ValueError):
        H._validate_init(("normal", 0.0))
    with pytest.raises(ValueError):
        H.BaselineSpec(name="x", metal_function="f", threadgroup=(0, 1, 1), input_bindings=(0,),
                       outputs=[])
    with pytest.raises(ValueError):
        H.BaselineSpec(name="x", metal_function="f", threadgroup=(1, 1, 1), input_bindings=(0, 0),
                       outputs=[])
    with pytest.raises(ValueError):
        H.Output(binding=40, dtype="f32", shape=(1,))
    with pytest.raises(ValueError):
        H.Scalar(binding=1, dtype="bf16", value=1)


def test_chip_override_mechanism(monkeypatch):
    monkeypatch.setattr(H, "_load_tuning", lambda: {("sqr_mm", "gfx950"): {"grid": (1, 2, 3)}})
    b = H.load_baseline("sqr_mm")
    m = H.build_manifest(b, b.make_inputs(0), warmup=1, iters=1, chip_type="gfx950:sramecc+")
    assert m["grid"] == [1, 2, 3]
    assert H.bucket_key_from_name("AMD Instinct MI355X") == "amd-instinct-mi355x"


# ---- the Model specs agree with the float64 oracle on small shapes -------------------------

def _load_model(name, **kw):
    b = H.load_baseline(name)
    return b.module.Model(**kw)


def test_matmul_models_match_oracle():
    a, c = torch.randn(33, 65), torch.randn(65, 17)
    for name in ("sqr_mm", "rect_mm"):
        got = _load_model(name).forward(a, c).numpy()
        assert np.allclose(got, oracle.matmul(a.numpy(), c.numpy()), rtol=1e-5, atol=1e-5)
    # large_mm's spec is the bf16 product: the fp32-accumulated sum rounded to
    # bf16 once, i.e. within half a bf16 ulp (2^-8 relative) of the exact product
    ab, cb = a.to(torch.bfloat16), c.to(torch.bfloat16)
    got = _load_model("large_mm").forward(ab, cb)
    assert got.dtype == torch.bfloat16
    exact = oracle.matmul(oracle.as_f64(ab), oracle.as_f64(cb))
    assert np.all(np.abs(oracle.as_f64(got) - exact) <= 2.0 ** -8 * np.abs(exact) * 1.0001 + 1e-6)


def test_transpose_model_matches_oracle():
    a = torch.randn(17, 29)
    assert np.array_equal(_load_model("transpose_2d").forward(a).numpy(), oracle.transpose(a.numpy()))


@pytest.mark.parametrize("pad,stride", [(1, 1), (0, 1), (1, 2)])
def test_conv_model_matches_oracle(pad, stride):
    x, w = torch.randn(2, 9, 10, 8), torch.randn(5, 3, 3, 8)
    got = _load_model("conv2d", in_channels=8, out_channels=5, stride=stride,
                      padding=pad).forward(x, w).numpy()
    want = oracle.conv2d_nhwc(x.numpy(), w.numpy(), stride, pad)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)


def test_decoder_step_model_matches_oracle():
    B, D, Hq, Hkv, FF, L = 3, 256, 2, 1, 384, 19
    Dh = D // Hq
    g = torch.Generator().manual_seed(5)
    mk = lambda *s, std=1.0: (torch.randn(*s, generator=g) * std).to(torch.bfloat16)  # noqa: E731
    ins = [mk(B, D), mk(D, D + 2 * Hkv * Dh, std=0.02), mk(D, D, std=0.02), mk(D, 2 * FF, std=0.02),
           mk(FF, D, std=0.02), mk(B, Hkv, L, Dh), mk(B, Hkv, L, Dh)]
    model = _load_model("llama_decoder_step", B=B, D=D, H=Hq, H_kv=Hkv, FF=FF, L=L)
    y, k, v = model.forward(*ins)
    wy, wk, wv = oracle.llama_decoder_step(*[oracle.as_f64(t) for t in ins], n_heads=Hq,
                                           n_kv_heads=Hkv)
    for got, want in ((y, wy), (k, wk), (v, wv)):
        assert np.allclose(got.numpy(), want, rtol=1e-4, atol=1e-4)

"""Pins the CPU oracle (oracle/) before anything is checked against it.

The reference ships no golden vectors for these kernels and MLX (its
arithmetic) is not installed, so each oracle function is pinned by checks
that do not restate its own formula: brute-force loops, a library routine
(torch float64 conv2d, scipy's expit, numpy complex arithmetic), closed forms
and invariants, chosen so that a dropped term, a wrong sign/index or a
transposed operand fails at least one of them.  A deliberately broken variant
of the oracle is shown to fail these checks (planted mistakes, end of file)."""
import inspect
import math

import numpy as np
import pytest
import scipy.special
import torch

import oracle

RNG = np.random.default_rng(1234)


def rnd(*shape):
    return RNG.standard_normal(shape)


# ---- bf16 conversion -----------------------------------------------------------------

def test_bf16_round_trip_and_rne():
    x = np.array([1.0, -2.5, 3.140625, 0.0, -0.0, np.inf, -np.inf], np.float32)
    assert np.array_equal(oracle.bf16_bits_to_f64(oracle.f32_to_bf16_bits(x)), x.astype(np.float64))
    # 1 + 2^-8 is exactly half way between bf16 neighbours 1 and 1 + 2^-7: ties to even -> 1
    assert oracle.bf16_bits_to_f64(oracle.f32_to_bf16_bits(np.float32(1 + 2**-8)))[()] == 1.0
    # 1 + 3*2^-8 is half way between 1 + 2^-7 and 1 + 2^-6: ties to even -> 1 + 2^-6
    assert oracle.bf16_bits_to_f64(oracle.f32_to_bf16_bits(np.float32(1 + 3 * 2**-8)))[()] == 1 + 2**-6
    assert np.isnan(oracle.bf16_bits_to_f64(oracle.f32_to_bf16_bits(np.float32(np.nan))))


def test_bf16_matches_torch_conversion():
    x = (RNG.standard_normal(10000) * 10).astype(np.float32)
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16_bits(x), t)


# ---- transpose -------------------------------------------------------------------------

def test_transpose_index_identity():
    a = rnd(37, 53).astype(np.float32)
    b = oracle.transpose(a)
    assert b.shape == (53, 37)
    for i in range(37):
        for j in range(53):
            assert b[j, i] == a[i, j]


def test_transpose_involution_and_c_restatement():
    a = rnd(129, 67).astype(np.float32)
    assert np.array_equal(oracle.transpose(oracle.transpose(a)), a)
    out = np.empty((67, 129), np.float32)
    oracle.cref().oracle_transpose_f32(a.ctypes.data, out.ctypes.data, 129, 67)
    assert np.array_equal(out, oracle.transpose(a))


# ---- matmul ------------------------------------------------------------------------------

def test_matmul_brute_force():
    a, b = rnd(5, 7), rnd(7, 3)
    c = oracle.matmul(a, b)
    for i in range(5):
        for j in range(3):
            assert np.isclose(c[i, j], sum(a[i, p] * b[p, j] for p in range(7)), rtol=1e-13)


def test_matmul_identity_permutation_zero():
    a = rnd(16, 16)
    assert np.array_equal(oracle.matmul(a, np.eye(16)), a)
    perm = np.eye(16)[RNG.permutation(16)]
    assert np.array_equal(oracle.matmul(perm, a), a[np.argmax(perm, axis=1)])
    assert not oracle.matmul(a, np.zeros((16, 4))).any()


def test_matmul_rank1_closed_form():
    u, v, w, z = rnd(9), rnd(6), rnd(6), rnd(4)
    got = oracle.matmul(np.outer(u, v), np.outer(w, z))
    assert np.allclose(got, np.dot(v, w) * np.outer(u, z), rtol=1e-12, atol=1e-12)


def test_matmul_matches_c_triple_loop():
    a, b = rnd(33, 70), rnd(70, 41)
    c = np.empty((33, 41))
    oracle.cref().oracle_gemm_f64(a.ctypes.data, b.ctypes.data, c.ctypes.data, 33, 41, 70)
    assert np.allclose(oracle.matmul(a, b), c, rtol=1e-12, atol=1e-12)


# ---- conv2d -------------------------------------------------------------------------------

def _torch_conv(x, w, stride, pad):
    y = torch.nn.functional.conv2d(torch.from_numpy(x).permute(0, 3, 1, 2),
                                   torch.from_numpy(w).permute(0, 3, 1, 2),
                                   stride=stride, padding=pad)
    return y.permute(0, 2, 3, 1).numpy()


@pytest.mark.parametrize("n,h,w,c,o,r,s,st,pad", [
    (2, 9, 11, 3, 4, 3, 3, 1, 1), (1, 8, 8, 5, 2, 3, 3, 1, 0), (2, 7, 6, 4, 3, 3, 3, 2, 1),
    (1, 5, 5, 2, 2, 1, 1, 1, 0), (1, 6, 9, 3, 5, 3, 2, 1, 2),
])
def test_conv2d_vs_torch_and_c(n, h, w, c, o, r, s, st, pad):
    x, wt = rnd(n, h, w, c), rnd(o, r, s, c)
    want = _torch_conv(x, wt, st, pad)
    got = oracle.conv2d_nhwc(x, wt, st, pad)
    assert got.shape == want.shape
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    yc = np.empty(want.shape)
    oracle.cref().oracle_conv2d_nhwc_f64(x.ctypes.data, wt.ctypes.data, yc.ctypes.data,
                                         n, h, w, c, o, r, s, st, pad)
    assert np.allclose(got, yc, rtol=1e-12, atol=1e-12)


def test_conv2d_1x1_is_gemm():
    x, wt = rnd(2, 4, 5, 6), rnd(7, 1, 1, 6)
    got = oracle.conv2d_nhwc(x, wt, 1, 0)
    assert np.allclose(got, (x.reshape(-1, 6) @ wt.reshape(7, 6).T).reshape(2, 4, 5, 7))


def test_conv2d_delta_kernel_is_shifted_copy():
    # A 3x3 kernel that picks tap (r, s) = (0, 2) of channel 1 -> y[p, q] = x[p-1, q+1]
    # (zero outside), pad 1.
    x = rnd(1, 6, 7, 3)
    wt = np.zeros((1, 3, 3, 3))
    wt[0, 0, 2, 1] = 1.0
    y = oracle.conv2d_nhwc(x, wt, 1, 1)[0, :, :, 0]
    want = np.zeros((6, 7))
    want[1:, :-1] = x[0, :-1, 1:, 1]
    assert np.array_equal(y, want)


# ---- decoder pieces ------------------------------------------------------------------------

def test_rms_norm_closed_forms():
    c = 3.0
    x = np.full((2, 8), c)
    assert np.allclose(oracle.rms_norm(x, 1e-5), c / np.sqrt(c * c + 1e-5))
    y = oracle.rms_norm(rnd(4, 4096), 0.0)
    assert np.allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, atol=1e-12)


def test_rope_identity_norm_composition_complex():
    t = rnd(3, 5, 128)
    base = 500000.0
    assert np.allclose(oracle.rope_interleaved(t, 0, base), t)
    r = oracle.rope_interleaved(t, 2048, base)
    pair_norm = lambda a: a[..., 0::2] ** 2 + a[..., 1::2] ** 2  # noqa: E731
    assert np.allclose(pair_norm(r), pair_norm(t))
    assert np.allclose(oracle.rope_interleaved(oracle.rope_interleaved(t, 100, base), 1948, base),
                       r, atol=1e-9)
    # complex form: (t0 + i t1) * exp(i pos w_k), w_k = base^(-2k/Dh)
    w = base ** (-2.0 * np.arange(64) / 128)
    z = (t[..., 0::2] + 1j * t[..., 1::2]) * np.exp(1j * 2048 * w)
    assert np.allclose(r[..., 0::2], z.real) and np.allclose(r[..., 1::2], z.imag)


def test_rope_per_position_broadcast():
    t = rnd(2, 6, 8)
    pos = np.arange(6)[None, :]
    r = oracle.rope_interleaved(t, pos, 10000.0)
    for p in range(6):
        assert np.allclose(r[:, p], oracle.rope_interleaved(t[:, p], p, 10000.0))


def test_silu_matches_expit():
    v = np.linspace(-30, 30, 1001)
    assert np.allclose(oracle.silu(v), v * scipy.special.expit(v), rtol=1e-12, atol=1e-300)
    assert oracle.silu(np.array(0.0)) == 0.0


def test_attention_single_key_equal_keys_and_mha():
    b, h, hkv, dh = 2, 4, 2, 16
    q = rnd(b, h, dh)
    empty = np.zeros((b, hkv, 0, dh))
    k_new, v_new = rnd(b, hkv, dh), rnd(b, hkv, dh)
    out = oracle.gqa_decode_attention(q, empty, empty, k_new, v_new)
    assert np.allclose(out, np.repeat(v_new, h // hkv, axis=1))           # one key -> its value
    k_same = np.repeat(k_new[:, :, None], 5, axis=2)
    v_cache = rnd(b, hkv, 5, dh)
    out = oracle.gqa_decode_attention(q, k_same, v_cache, k_new, v_new)
    mean_v = (v_cache.sum(axis=2) + v_new) / 6.0                          # equal scores -> mean
    assert np.allclose(out, np.repeat(mean_v, h // hkv, axis=1))
    # G = 1: brute-force multi-head softmax
    kc, vc = rnd(b, h, 7, dh), rnd(b, h, 7, dh)
    kn, vn = rnd(b, h, dh), rnd(b, h, dh)
    out = oracle.gqa_decode_attention(q, kc, vc, kn, vn)
    for i in range(b):
        for j in range(h):
            keys = np.vstack([kc[i, j], kn[i, j]])
            vals = np.vstack([vc[i, j], vn[i, j]])
            s = keys @ q[i, j] / np.sqrt(dh)
            p = np.exp(s - s.max())
            p /= p.sum()
            assert np.allclose(out[i, j], p @ vals)


def test_attention_head_maps_to_kv_head_h_div_g():
    b, h, hkv, dh, L = 1, 8, 2, 4, 3
    q = rnd(b, h, dh)
    kc = rnd(b, hkv, L, dh)
    vc = np.zeros((b, hkv, L, dh))
    for j in range(hkv):
        vc[:, j] = j + 1.0                       # every value of kv head j equals j + 1
    kn = rnd(b, hkv, dh)
    vn = np.stack([np.full((b, dh), j + 1.0) for j in range(hkv)], axis=1)
    out = oracle.gqa_decode_attention(q, kc, vc, kn, vn)
    for hh in range(h):
        assert np.allclose(out[0, hh], hh // (h // hkv) + 1.0)


def _decoder_inputs(b, d, h, hkv, ff, L, scale=0.02):
    dh = d // h
    return dict(x=rnd(b, d), w_qkv=rnd(d, d + 2 * hkv * dh) * scale, w_o=rnd(d, d) * scale,
                w_gu=rnd(d, 2 * ff) * scale, w_down=rnd(ff, d) * scale,
                k_cache=rnd(b, hkv, L, dh), v_cache=rnd(b, hkv, L, dh))


def test_decoder_step_zero_weights_is_identity():
    a = _decoder_inputs(2, 64, 4, 2, 96, 5)
    for k in ("w_qkv", "w_o", "w_gu", "w_down"):
        a[k] = np.zeros_like(a[k])
    y, kn, vn = oracle.llama_decoder_step(**a, n_heads=4, n_kv_heads=2)
    assert np.array_equal(y, a["x"]) and not kn.any() and not vn.any()


def test_decoder_step_empty_cache_equals_single_token_prefill():
    # With no cached positions the new token sits at position 0 and attends to
    # itself only: exactly the reference's prefill layer with S = 1.
    a = _decoder_inputs(3, 64, 4, 2, 96, 0, scale=0.1)
    y, _, _ = oracle.llama_decoder_step(**a, n_heads=4, n_kv_heads=2, base=10000.0)
    for i in range(3):
        yp = oracle.llama_decoder_layer(a["x"][i:i + 1], a["w_qkv"], a["w_o"], a["w_gu"],
                                        a["w_down"], n_heads=4, n_kv_heads=2, base=10000.0)
        assert np.allclose(y[i], yp[0], rtol=1e-12, atol=1e-12)


def test_decoder_step_new_key_is_rotated_projection():
    a = _decoder_inputs(2, 64, 4, 2, 32, 6, scale=0.1)
    _, kn, vn = oracle.llama_decoder_step(**a, n_heads=4, n_kv_heads=2)
    h = a["x"] / np.sqrt(np.mean(a["x"] ** 2, axis=-1, keepdims=True) + 1e-5)
    kv = h @ a["w_qkv"][:, 64:]
    assert np.allclose(vn.reshape(2, -1), kv[:, 32:])
    # undo the rotation with the complex conjugate at position L = 6
    w = 500000.0 ** (-2.0 * np.arange(8) / 16)
    z = (kn[..., 0::2] + 1j * kn[..., 1::2]) * np.exp(-1j * 6 * w)
    k = np.empty_like(kn)
    k[..., 0::2], k[..., 1::2] = z.real, z.imag
    assert np.allclose(k.reshape(2, -1), kv[:, :32])


def test_decoder_layer_zero_weights_is_identity():
    x = rnd(8, 32)
    z = lambda *s: np.zeros(s)  # noqa: E731
    y = oracle.llama_decoder_layer(x, z(32, 64), z(32, 32), z(32, 96), z(48, 32),
                                   n_heads=4, n_kv_heads=2)
    assert np.array_equal(y, x)


# ---- the FFN half and the whole decoder against pure-Python loops --------------------------
# Written from reference mlx/kernels/full/llama_decoder_layer.py:24-64 with
# `math` only: h = rmsnorm(x) (:48-50); q|k|v = h W_qkv, columns [Q | K | V];
# RoPE on pairs (2i, 2i+1) at angle pos * base^(-2i/Dh) (:52-64); query head h
# reads kv head h // G (:34); softmax(q k / sqrt(Dh)) v; x1 = x + attn W_o;
# h2 = rmsnorm(x1); y = x1 + (silu(h2 W_gate) * h2 W_up) W_down, W_gu columns
# [gate | up] (:41-46), silu(v) = v / (1 + e^-v).

def _rot(vec, pos, base):
    out = list(vec)
    for i in range(len(vec) // 2):
        a = pos / base ** (2.0 * i / len(vec))
        out[2 * i] = vec[2 * i] * math.cos(a) - vec[2 * i + 1] * math.sin(a)
        out[2 * i + 1] = vec[2 * i] * math.sin(a) + vec[2 * i + 1] * math.cos(a)
    return out


def _loop_ffn(x1, w_gu, w_down, eps):
    """Rows of x1 (the attention half's output) through the FFN half."""
    d, ff = len(x1[0]), len(w_down)
    out = []
    for row in x1:
        h2 = _brute_rms_row(list(row), eps)
        act = []
        for f in range(ff):
            g = sum(h2[k] * w_gu[k][f] for k in range(d))
            u = sum(h2[k] * w_gu[k][ff + f] for k in range(d))
            act.append(g / (1.0 + math.exp(-g)) * u)
        out.append([row[j] + sum(act[f] * w_down[f][j] for f in range(ff)) for j in range(d)])
    return np.array(out)


def _loop_decoder_step(x, w_qkv, w_o, w_gu, w_down, k_cache, v_cache, H, HKV, base, eps,
                       dh=None):
    """One new token per sequence at position L attending to the L cached
    (already rotated) keys and itself.  The attention width QD = H * dh is D
    unless dh is given (one tensor-parallel shard: W_o has QD rows)."""
    B, D = x.shape
    dh = D // H if dh is None else dh
    QD, g, L = H * dh, H // HKV, k_cache.shape[2]
    x1, k_new, v_new = [], np.zeros((B, HKV, dh)), np.zeros((B, HKV, dh))
    for b in range(B):
        h = _brute_rms_row(list(x[b]), eps)
        qkv = [sum(h[k] * w_qkv[k, j] for k in range(D)) for j in range(w_qkv.shape[1])]
        for kvh in range(HKV):
            k_new[b, kvh] = _rot(qkv[QD + kvh * dh:QD + (kvh + 1) * dh], L, base)
            v_new[b, kvh] = qkv[QD + (HKV + kvh) * dh:QD + (HKV + kvh + 1) * dh]
        att = [0.0] * QD
        for hh in range(H):
            kvh = hh // g
            q = _rot(qkv[hh * dh:(hh + 1) * dh], L, base)
            keys = [list(k_cache[b, kvh, j]) for j in range(L)] + [list(k_new[b, kvh])]
            vals = [list(v_cache[b, kvh, j]) for j in range(L)] + [list(v_new[b, kvh])]
            sc = [sum(qi * ki for qi, ki in zip(q, key)) / math.sqrt(dh) for key in keys]
            mx = max(sc)
            e = [math.exp(s - mx) for s in sc]
            z = sum(e)
            for dd in range(dh):
                att[hh * dh + dd] = sum(e[j] / z * vals[j][dd] for j in range(L + 1))
        x1.append([x[b, j] + sum(att[k] * w_o[k, j] for k in range(QD)) for j in range(D)])
    return _loop_ffn(x1, w_gu, w_down, eps), k_new, v_new


def _step_inputs(seed=7, B=2, D=16, H=4, HKV=2, FF=6, L=3, scale=0.4):
    r = np.random.default_rng(seed)
    dh = D // H
    n = lambda *s: r.standard_normal(s)  # noqa: E731
    return dict(x=n(B, D), w_qkv=n(D, D + 2 * HKV * dh) * scale, w_o=n(D, D) * scale,
                w_gu=n(D, 2 * FF) * scale, w_down=n(FF, D) * scale,
                k_cache=n(B, HKV, L, dh), v_cache=n(B, HKV, L, dh))


def _step_matches_loops(step_fn, a, H=4, HKV=2, base=500000.0, eps=1e-5, dh=None):
    kw = {} if dh is None else {"head_dim": dh}
    y, kn, vn = step_fn(**a, n_heads=H, n_kv_heads=HKV, base=base, eps=eps, **kw)
    wy, wk, wv = _loop_decoder_step(*(a[k] for k in ("x", "w_qkv", "w_o", "w_gu", "w_down",
                                                     "k_cache", "v_cache")), H, HKV, base, eps,
                                    dh)
    return (np.allclose(y, wy, rtol=1e-10, atol=1e-10) and np.allclose(kn, wk, rtol=1e-10, atol=1e-10)
            and np.allclose(vn, wv, rtol=1e-10, atol=1e-10))


def _layer_matches_loops(layer_fn, x, wqkv, wo, wgu, wd, H=4, HKV=2, base=100.0, eps=1e-5):
    got = layer_fn(x, wqkv, wo, wgu, wd, n_heads=H, n_kv_heads=HKV, base=base, eps=eps)
    h = np.array([_brute_rms_row(list(row), eps) for row in x])
    x1 = x + _brute_attention(h, wqkv, wo, H, HKV, base)
    return np.allclose(got, _loop_ffn(x1, wgu, wd, eps), rtol=1e-10, atol=1e-10)


def test_decoder_step_matches_loops():
    # every weight non-zero, big enough that silu, softmax and RoPE are far from linear
    assert _step_matches_loops(oracle.llama_decoder_step, _step_inputs())
    assert _step_matches_loops(oracle.llama_decoder_step, _step_inputs(seed=8, H=4, HKV=1, L=5),
                               HKV=1, base=10000.0)


def test_decoder_step_tensor_parallel_shard_matches_loops():
    """One shard of a layer (attention width QD = H * Dh < D: its heads, its
    QD rows of W_o) against the loop restatement, and the whole-layer width
    (head_dim = D / H given explicitly) identical to the default."""
    r = np.random.default_rng(11)
    B, D, H, HKV, DH, FF, L = 2, 16, 2, 1, 4, 6, 3
    QD = H * DH
    n = lambda *s: r.standard_normal(s)  # noqa: E731
    a = dict(x=n(B, D), w_qkv=n(D, QD + 2 * HKV * DH) * 0.4, w_o=n(QD, D) * 0.4,
             w_gu=n(D, 2 * FF) * 0.4, w_down=n(FF, D) * 0.4,
             k_cache=n(B, HKV, L, DH), v_cache=n(B, HKV, L, DH))
    assert _step_matches_loops(oracle.llama_decoder_step, a, H=H, HKV=HKV, dh=DH)
    full = _step_inputs()
    y0, k0, v0 = oracle.llama_decoder_step(**full, n_heads=4, n_kv_heads=2)
    y1, k1, v1 = oracle.llama_decoder_step(**full, n_heads=4, n_kv_heads=2, head_dim=4)
    assert np.array_equal(y0, y1) and np.array_equal(k0, k1) and np.array_equal(v0, v1)


def test_decoder_step_ffn_half_with_zero_w_o():
    # W_o = 0 makes x1 = x, so y is the FFN half of x alone; compared with loops
    a = _decoder_inputs(2, 64, 4, 2, 96, 5, scale=0.2)
    a["w_o"] = np.zeros_like(a["w_o"])
    y, _, _ = oracle.llama_decoder_step(**a, n_heads=4, n_kv_heads=2)
    assert np.allclose(y, _loop_ffn(a["x"], a["w_gu"], a["w_down"], 1e-5), rtol=1e-10, atol=1e-10)


def test_decoder_layer_ffn_half_with_zero_w_qkv():
    # W_qkv = 0 makes v = 0, hence attention = 0 and x1 = x
    x, D, FF = rnd(5, 32), 32, 48
    wgu, wd = rnd(D, 2 * FF) * 0.3, rnd(FF, D) * 0.3
    y = oracle.llama_decoder_layer(x, np.zeros((D, 64)), rnd(D, D), wgu, wd, n_heads=4, n_kv_heads=2)
    assert np.allclose(y, _loop_ffn(x, wgu, wd, 1e-5), rtol=1e-10, atol=1e-10)


def test_decoder_layer_matches_loops():
    S, D, H, HKV, FF = 3, 16, 4, 2, 6
    x, wqkv, wo = rnd(S, D), rnd(D, D + 2 * HKV * (D // H)) * 0.4, rnd(D, D) * 0.4
    wgu, wd = rnd(D, 2 * FF) * 0.4, rnd(FF, D) * 0.4
    assert _layer_matches_loops(oracle.llama_decoder_layer, x, wqkv, wo, wgu, wd)


# ---- decoder sub-ops at the reference shapes ---------------------------------------------

def test_fused_add_rms_norm_closed_forms():
    x, r = rnd(5, 16), rnd(5, 16)
    assert np.allclose(oracle.fused_add_rms_norm(x, np.zeros_like(x), 1e-5), oracle.rms_norm(x, 1e-5))
    assert np.array_equal(oracle.fused_add_rms_norm(x, -x, 1e-5), np.zeros_like(x))
    # commutes in its two inputs, and unit output RMS when eps is negligible
    assert np.allclose(oracle.fused_add_rms_norm(x, r, 0.0), oracle.fused_add_rms_norm(r, x, 0.0))
    y = oracle.fused_add_rms_norm(x, r, 0.0)
    assert np.allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0)


def _brute_rms_row(row, eps):
    ms = sum(v * v for v in row) / len(row)
    return [v / (ms + eps) ** 0.5 for v in row]


def test_rms_norm_linear_identity_and_brute_force():
    x = rnd(3, 6)
    assert np.allclose(oracle.rms_norm_linear(x, np.eye(6), 1e-5), oracle.rms_norm(x, 1e-5))
    w = rnd(4, 6)   # [out][in]
    got = oracle.rms_norm_linear(x, w, 1e-5)
    for i in range(3):
        n = _brute_rms_row(list(x[i]), 1e-5)
        for o in range(4):
            assert abs(got[i, o] - sum(n[k] * w[o, k] for k in range(6))) < 1e-12


def test_swiglu_zero_weights_and_brute_force():
    x, wg, wu = rnd(3, 5), rnd(5, 4), rnd(5, 4)
    assert np.array_equal(oracle.swiglu(x, wg, np.zeros_like(wu)), np.zeros((3, 4)))
    assert np.array_equal(oracle.swiglu(x, np.zeros_like(wg), wu), np.zeros((3, 4)))
    got = oracle.swiglu(x, wg, wu)
    for i in range(3):
        for j in range(4):
            g = sum(x[i, k] * wg[k, j] for k in range(5))
            u = sum(x[i, k] * wu[k, j] for k in range(5))
            assert abs(got[i, j] - g * scipy.special.expit(g) * u) < 1e-12


def test_rope_embedding_rows_at_positions():
    x = rnd(6, 8)
    y = oracle.rope_embedding(x, 10000.0)
    assert np.array_equal(y[0], x[0])                       # position 0: identity
    for p in range(6):                                      # complex multiply, omega = 1/base^(2i/D)
        w = 1.0 / 10000.0 ** (2.0 * np.arange(4) / 8)
        z = (x[p, 0::2] + 1j * x[p, 1::2]) * np.exp(1j * p * w)
        assert np.allclose(y[p, 0::2], z.real) and np.allclose(y[p, 1::2], z.imag)


def _brute_attention(x, w_qkv, w_o, H, HKV, base):
    """Pure-Python loops: every head, query and key, math.exp softmax."""
    import math
    S, D = x.shape
    dh, g = D // H, H // HKV
    qkv = [[sum(x[i, k] * w_qkv[k, j] for k in range(D)) for j in range(w_qkv.shape[1])]
           for i in range(S)]

    def rot(vec, pos):
        out = list(vec)
        for i in range(len(vec) // 2):
            a = pos / base ** (2.0 * i / len(vec))
            out[2 * i] = vec[2 * i] * math.cos(a) - vec[2 * i + 1] * math.sin(a)
            out[2 * i + 1] = vec[2 * i] * math.sin(a) + vec[2 * i + 1] * math.cos(a)
        return out

    att = [[0.0] * D for _ in range(S)]
    for h in range(H):
        kvh = h // g
        for i in range(S):
            q = rot(qkv[i][h * dh:(h + 1) * dh], i)
            sc = []
            for j in range(S):
                k = rot(qkv[j][D + kvh * dh:D + (kvh + 1) * dh], j)
                sc.append(sum(a * b for a, b in zip(q, k)) / math.sqrt(dh))
            mx = max(sc)
            e = [math.exp(v - mx) for v in sc]
            z = sum(e)
            for d in range(dh):
                att[i][h * dh + d] = sum(e[j] / z * qkv[j][D + (HKV + kvh) * dh + d]
                                         for j in range(S))
    return np.array([[sum(att[i][k] * w_o[k, j] for k in range(D)) for j in range(D)]
                     for i in range(S)])


def test_llama_attention_brute_force_and_single_token():
    S, D, H, HKV = 3, 8, 4, 2
    x, wqkv, wo = rnd(S, D), rnd(D, D + 2 * HKV * (D // H)), rnd(D, D)
    got = oracle.llama_attention(x, wqkv, wo, n_heads=H, n_kv_heads=HKV, base=100.0)
    assert np.allclose(got, _brute_attention(x, wqkv, wo, H, HKV, 100.0), rtol=1e-10, atol=1e-10)
    # one token: softmax over one key is 1, RoPE at position 0 is the identity,
    # so every head h outputs v of kv head h // G and y = that @ W_o
    x1 = x[:1]
    v = (x1 @ wqkv)[:, D + HKV * 2:]
    heads = np.concatenate([v[:, (h // (H // HKV)) * 2:(h // (H // HKV)) * 2 + 2] for h in range(H)], 1)
    assert np.allclose(oracle.llama_attention(x1, wqkv, wo, n_heads=H, n_kv_heads=HKV), heads @ wo)


def test_llama_attention_is_the_decoder_layers_attention_half():
    S, D, H, HKV, FF = 5, 16, 4, 2, 8
    x, wqkv, wo = rnd(S, D), rnd(D, D + 2 * HKV * (D // H)), rnd(D, D)
    zero_gu, zero_dn = np.zeros((D, 2 * FF)), np.zeros((FF, D))
    layer = oracle.llama_decoder_layer(x, wqkv, wo, zero_gu, zero_dn, n_heads=H, n_kv_heads=HKV)
    attn = oracle.llama_attention(oracle.rms_norm(x, 1e-5), wqkv, wo, n_heads=H, n_kv_heads=HKV)
    assert np.allclose(layer, x + attn)


def test_matvec_and_batch_mm():
    a, v = rnd(4, 5), rnd(5)
    assert np.allclose(oracle.matmul(a, v), [sum(a[i, k] * v[k] for k in range(5)) for i in range(4)])
    A, B = rnd(3, 2, 4), rnd(3, 4, 5)
    got = oracle.matmul(A, B)
    for b in range(3):
        assert np.allclose(got[b], oracle.matmul(A[b], B[b]))


# ---- planted mistakes: the checks above must catch plausible oracle bugs -----------------

def test_planted_mistakes_are_caught(monkeypatch):
    t = rnd(1, 1, 128)
    r = oracle.rope_interleaved(t, 5, 10000.0)
    # wrong sign in the rotation
    bad = r.copy()
    bad[..., 1::2] = t[..., 0::2] * np.sin(5 * 10000.0 ** (-2 * np.arange(64) / 128)) * -1 + \
        t[..., 1::2] * np.cos(5 * 10000.0 ** (-2 * np.arange(64) / 128))
    w = 10000.0 ** (-2.0 * np.arange(64) / 128)
    z = (t[..., 0::2] + 1j * t[..., 1::2]) * np.exp(1j * 5 * w)
    assert not np.allclose(bad[..., 1::2], z.imag)
    # transposed weight operand in conv
    x, wt = rnd(1, 5, 5, 3), rnd(3, 3, 3, 3)
    wrong = oracle.conv2d_nhwc(x, np.swapaxes(wt, 1, 2), 1, 1)
    assert not np.allclose(wrong, _torch_conv(x, wt, 1, 1))
    # GQA with head h -> kv head h % Hkv instead of h // G
    b, h, hkv, dh = 1, 4, 2, 4
    q = rnd(b, h, dh)
    vc = np.stack([np.full((b, 2, dh), j + 1.0) for j in range(hkv)], axis=1)
    kc = rnd(b, hkv, 2, dh)
    kn = rnd(b, hkv, dh)
    vn = vc[:, :, 0]
    modulo = np.array([oracle.gqa_decode_attention(q[:, [hh]], kc[:, [hh % hkv]], vc[:, [hh % hkv]],
                                                   kn[:, [hh % hkv]], vn[:, [hh % hkv]])[0, 0, 0]
                       for hh in range(h)])
    assert not np.allclose(modulo, [hh // (h // hkv) + 1.0 for hh in range(h)])


# Mutation checks: one plausible mistake planted in a copy of the oracle's own
# source (exec'd in the oracle module's namespace) must fail the loop checks.
def _mutant(fn, old, new):
    src = inspect.getsource(fn)
    assert src.count(old) == 1, f"mutation site {old!r} not found once in {fn.__name__}"
    ns = dict(vars(oracle.oracle))
    exec(compile(src.replace(old, new), "<mutant>", "exec"), ns)
    return ns[fn.__name__]


STEP_MUTATIONS = [
    # gate and up halves swapped, i.e. silu on the up half
    ("silu(gu[:, :ff_dim]) * gu[:, ff_dim:]", "silu(gu[:, ff_dim:]) * gu[:, :ff_dim]"),
    ("silu(gu[:, :ff_dim]) * gu[:, ff_dim:]", "gu[:, :ff_dim] * gu[:, ff_dim:]"),         # no silu
    ("silu(gu[:, :ff_dim]) * gu[:, ff_dim:]", "silu(gu[:, :ff_dim] * gu[:, ff_dim:])"),   # silu last
    ("h2 = rms_norm(x1, eps)", "h2 = rms_norm(x, eps)"),          # FFN normalises x, not x1
    ("y = x1 + act @", "y = x + act @"),                          # FFN residual from x
    ("x1 = x + attn", "x1 = attn"),                               # attention residual dropped
    ("q = rope_interleaved(q, pos, base)", "q = q"),              # q not rotated
]


@pytest.mark.parametrize("old,new", STEP_MUTATIONS)
def test_planted_decoder_step_mistakes_are_caught(old, new):
    assert not _step_matches_loops(_mutant(oracle.llama_decoder_step, old, new), _step_inputs())


LAYER_MUTATIONS = [
    ("(silu(gu[:, :ff_dim]) * gu[:, ff_dim:])", "(silu(gu[:, ff_dim:]) * gu[:, :ff_dim])"),
    ("(silu(gu[:, :ff_dim]) * gu[:, ff_dim:])", "(gu[:, :ff_dim] * gu[:, ff_dim:])"),
    ("h2 = rms_norm(x1, eps)", "h2 = rms_norm(x, eps)"),
    ("return x1 + (", "return x + ("),
]


@pytest.mark.parametrize("old,new", LAYER_MUTATIONS)
def test_planted_decoder_layer_mistakes_are_caught(old, new):
    r = np.random.default_rng(3)
    S, D, H, HKV, FF = 3, 16, 4, 2, 6
    args = (r.standard_normal((S, D)), r.standard_normal((D, D + 2 * HKV * (D // H))) * 0.4,
            r.standard_normal((D, D)) * 0.4, r.standard_normal((D, 2 * FF)) * 0.4,
            r.standard_normal((FF, D)) * 0.4)
    assert _layer_matches_loops(oracle.llama_decoder_layer, *args)
    assert not _layer_matches_loops(_mutant(oracle.llama_decoder_layer, old, new), *args)

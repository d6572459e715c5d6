"""CPU oracle for the kernel-registry hot path — TEST INFRASTRUCTURE ONLY.

float64 numpy restatements of the reference's MLX `Model.forward`s.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker (or the timed CPU baseline): nothing in
metalbench_amd/ imports it, and the GPU path never falls back to it.

Every function names the reference lines it restates.  The reference's own
arithmetic lives in MLX (requirements.txt:1, `mlx>=0.18.0`, unpinned and not
vendored), which is not installed here; the reference ships no golden vectors
or fixtures for these kernels (results/*.json keep only timings and max_err).
How each function is pinned (tests/test_oracle.py):
  transpose            index identity, involution, numpy's own transpose
  matmul               brute-force triple loop, identity/permutation/zero,
                       rank-1 closed form, the C restatement (oracle/cref.c)
  conv2d_nhwc          torch.nn.functional.conv2d in float64 (library routine),
                       direct 7-loop C restatement, 1x1 == GEMM, delta kernel ==
                       shifted copy with zero border
  rms_norm             constant-row closed form, unit output RMS
  rope_interleaved     identity at pos 0, pair-norm preservation, composition,
                       complex multiply (t0 + i t1) e^{i pos w}
  gqa_decode_attention single key -> v, equal keys -> mean(v), G=1 == brute-force
                       MHA, head h reads kv head h // G (distinct-valued heads)
  silu / swiglu        silu(0) = 0, scipy.special.expit form
  llama_decoder_step   pure-Python loops (math only) over the whole step with
                       every weight non-zero; W_o = 0 -> y = x + FFN(x) by
                       loops; zero weights -> y = x; L = 0 equals the S = 1
                       prefill; planted FFN/residual/RoPE mutations fail
  llama_decoder_layer  pure-Python loops over the whole layer; W_qkv = 0 ->
                       y = x + FFN(x) by loops; zero weights -> y = x;
                       planted FFN/residual mutations fail
  fused_add_rms_norm   residual 0 -> rms_norm(x); x = -residual -> 0
  rms_norm_linear      W = I -> rms_norm(x); brute-force loops
  swiglu               zero gate or up weights -> 0; brute-force loops
  llama_attention      S = 1 closed form (v @ W_o); brute-force per-head
                       loops; equals the decoder layer's attention half
  rope_embedding       rope_interleaved over rows at positions 0..S-1
  matvec / batch_mm    brute-force loops; per-batch 2-D matmul
"""
from __future__ import annotations

import numpy as np

# ---- bf16 <-> float ------------------------------------------------------------------


def bf16_bits_to_f64(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float64 (exact)."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32).astype(np.float64)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (NaN kept quiet)."""
    f = np.atleast_1d(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[np.isnan(f)] = 0x7FC0
    return r.reshape(np.shape(x))


def as_f64(t) -> np.ndarray:
    """torch tensor (f32 or bf16) or numpy array -> float64 numpy."""
    if hasattr(t, "detach"):
        import torch
        t = t.detach().cpu()
        if t.dtype == torch.bfloat16:
            return bf16_bits_to_f64(t.view(torch.int16).numpy().view(np.uint16))
        return t.numpy().astype(np.float64)
    a = np.asarray(t)
    if a.dtype == np.uint16:
        return bf16_bits_to_f64(a)
    return a.astype(np.float64)


# ---- common set -------------------------------------------------------------------------


def transpose(a: np.ndarray) -> np.ndarray:
    """B = A^T (reference mlx/kernels/common/transpose_2d.py:10-11)."""
    return np.ascontiguousarray(np.asarray(a).T)


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """C = A @ B in float64 (reference mlx/kernels/common/sqr_mm.py:10-11; the
    bf16 GEMM is the same product of bf16-valued operands)."""
    return np.asarray(a, np.float64) @ np.asarray(b, np.float64)


def conv2d_nhwc(x: np.ndarray, w: np.ndarray, stride: int = 1, pad: int = 0) -> np.ndarray:
    """y[n,p,q,o] = sum_{r,s,c} xpad[n, p*st + r, q*st + s, c] * w[o,r,s,c].

    Cross-correlation as mx.conv2d (reference mlx/kernels/common/conv2d.py:11-12),
    NHWC input, OHWI weight (the layout of reference registry.py:469-477 and the
    weight index w[o*K + (r*S + s)*C + c] of metal/kernels/common/conv2d/
    default.metal:99-116), zero padding `pad` on H and W."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    n, h, wd, c = x.shape
    o, r, s, c2 = w.shape
    assert c == c2
    xp = np.pad(x, ((0, 0), (pad, pad), (pad, pad), (0, 0)))
    p_out = (h + 2 * pad - r) // stride + 1
    q_out = (wd + 2 * pad - s) // stride + 1
    y = np.zeros((n, p_out, q_out, o), np.float64)
    for i in range(r):
        for j in range(s):
            patch = xp[:, i:i + stride * (p_out - 1) + 1:stride,
                       j:j + stride * (q_out - 1) + 1:stride, :]          # (n, P, Q, C)
            y += patch @ w[:, i, j, :].T                                  # (C, O)
    return y


# ---- decoder pieces (reference mlx/kernels/full/llama_decoder_layer.py) ----------------


def rms_norm(x: np.ndarray, eps: float) -> np.ndarray:
    """x * rsqrt(mean(x^2, -1) + eps), no gain (reference :48-50)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def rope_interleaved(t: np.ndarray, pos, base: float) -> np.ndarray:
    """Rotate pairs (2i, 2i+1) of the last axis by pos * base^(-2i/Dh)
    (reference :52-64).  `pos` broadcasts against t.shape[:-1]."""
    t = np.asarray(t, np.float64)
    dh = t.shape[-1]
    half = dh // 2
    omega = 1.0 / (base ** (2.0 * np.arange(half, dtype=np.float64) / dh))
    ang = np.asarray(pos, np.float64)[..., None] * omega
    c, s = np.cos(ang), np.sin(ang)
    t0, t1 = t[..., 0::2], t[..., 1::2]
    out = np.empty_like(t)
    out[..., 0::2] = t0 * c - t1 * s
    out[..., 1::2] = t0 * s + t1 * c
    return out


def softmax(z: np.ndarray, axis: int = -1) -> np.ndarray:
    z = z - np.max(z, axis=axis, keepdims=True)
    e = np.exp(z)
    return e / np.sum(e, axis=axis, keepdims=True)


def silu(v: np.ndarray) -> np.ndarray:
    """v / (1 + e^-v) (reference nn.silu at :42; metal default.metal:14)."""
    return v / (1.0 + np.exp(-v))


def gqa_decode_attention(q, k_cache, v_cache, k_new, v_new, n_valid=None):
    """softmax(q k^T / sqrt(Dh)) v for one new token per sequence.

    q [B, H, Dh]; caches [B, Hkv, Lalloc, Dh] (first n_valid positions used);
    k_new / v_new [B, Hkv, Dh] are appended as the last key/value.  Query head h
    reads kv head h // G, the mx.repeat(k, G, axis=0) semantics of reference :34."""
    q = np.asarray(q, np.float64)
    b, h, dh = q.shape
    hkv = k_cache.shape[1]
    g = h // hkv
    L = k_cache.shape[2] if n_valid is None else n_valid
    keys = np.concatenate([np.asarray(k_cache, np.float64)[:, :, :L],
                           np.asarray(k_new, np.float64)[:, :, None]], axis=2)
    vals = np.concatenate([np.asarray(v_cache, np.float64)[:, :, :L],
                           np.asarray(v_new, np.float64)[:, :, None]], axis=2)
    qg = q.reshape(b, hkv, g, dh)
    scores = qg @ np.swapaxes(keys, 2, 3) / np.sqrt(dh)                     # (B, Hkv, G, L+1)
    p = softmax(scores, axis=-1)
    return (p @ vals).reshape(b, h, dh)


def llama_decoder_step(x, w_qkv, w_o, w_gu, w_down, k_cache, v_cache, *, n_heads, n_kv_heads,
                       pos=None, base=500000.0, eps=1e-5, head_dim=None):
    """One decode step (reference :24-46 applied to one new token per sequence).

    x [B, D]; w_qkv [D, QD + 2*Hkv*Dh] columns [Q|K|V]; w_o [QD, D];
    w_gu [D, 2FF] columns [gate|up]; w_down [FF, D]; caches [B, Hkv, L, Dh]
    holding already-rotated keys of positions 0..L-1.  The new token sits at
    position L (or `pos`).  Returns (y [B, D], k_new [B, Hkv, Dh], v_new).

    QD = n_heads * Dh.  With the default Dh = D / n_heads, QD = D: the
    reference's layer.  A smaller QD (an explicit `head_dim`) is one
    tensor-parallel shard of a layer computed alone (its heads, its rows of
    W_o, its FF columns), i.e. the same formula with the shard's matrices and
    no all-reduce."""
    x = np.asarray(x, np.float64)
    b, d = x.shape
    dh = d // n_heads if head_dim is None else head_dim
    qd = n_heads * dh
    L = k_cache.shape[2]
    pos = L if pos is None else pos
    ff_dim = w_down.shape[0]

    h = rms_norm(x, eps)
    qkv = h @ np.asarray(w_qkv, np.float64)
    q = qkv[:, :qd].reshape(b, n_heads, dh)
    k = qkv[:, qd:qd + n_kv_heads * dh].reshape(b, n_kv_heads, dh)
    v = qkv[:, qd + n_kv_heads * dh:].reshape(b, n_kv_heads, dh)
    q = rope_interleaved(q, pos, base)
    k = rope_interleaved(k, pos, base)
    attn = gqa_decode_attention(q, k_cache, v_cache, k, v)
    x1 = x + attn.reshape(b, qd) @ np.asarray(w_o, np.float64)
    h2 = rms_norm(x1, eps)
    gu = h2 @ np.asarray(w_gu, np.float64)
    act = silu(gu[:, :ff_dim]) * gu[:, ff_dim:]
    y = x1 + act @ np.asarray(w_down, np.float64)
    return y, k, v


def llama_decoder_layer(x, w_qkv, w_o, w_gu, w_down, *, n_heads, n_kv_heads, base=10000.0,
                        eps=1e-5):
    """The reference's prefill layer, verbatim semantics (reference :24-46):
    S tokens at positions 0..S-1, full (non-causal) softmax attention."""
    x = np.asarray(x, np.float64)
    s_len, d = x.shape
    dh = d // n_heads
    g = n_heads // n_kv_heads
    ff_dim = w_down.shape[0]
    h = rms_norm(x, eps)
    qkv = h @ np.asarray(w_qkv, np.float64)
    q = qkv[:, :d].reshape(s_len, n_heads, dh).transpose(1, 0, 2)
    k = qkv[:, d:d + n_kv_heads * dh].reshape(s_len, n_kv_heads, dh).transpose(1, 0, 2)
    v = qkv[:, d + n_kv_heads * dh:].reshape(s_len, n_kv_heads, dh).transpose(1, 0, 2)
    pos = np.arange(s_len, dtype=np.float64)[None, :]
    q = rope_interleaved(q, pos, base)
    k = rope_interleaved(k, pos, base)
    k = np.repeat(k, g, axis=0)
    v = np.repeat(v, g, axis=0)
    scores = q @ np.swapaxes(k, 1, 2) / np.sqrt(dh)
    p = softmax(scores, axis=-1)
    out = (p @ v).transpose(1, 0, 2).reshape(s_len, d) @ np.asarray(w_o, np.float64)
    x1 = x + out
    h2 = rms_norm(x1, eps)
    gu = h2 @ np.asarray(w_gu, np.float64)
    return x1 + (silu(gu[:, :ff_dim]) * gu[:, ff_dim:]) @ np.asarray(w_down, np.float64)


# ---- decoder sub-ops at the reference's own shapes -----------------------------------


def fused_add_rms_norm(x, residual, eps: float = 1e-5) -> np.ndarray:
    """RMSNorm(x + residual), unit gain (reference
    mlx/kernels/standard/fused_add_rms_norm.py:11-12)."""
    return rms_norm(np.asarray(x, np.float64) + np.asarray(residual, np.float64), eps)


def rms_norm_linear(x, w, eps: float = 1e-5) -> np.ndarray:
    """rms_norm(x) @ w.T, w [out][in] (reference
    mlx/kernels/standard/rms_norm_linear.py:12-14)."""
    return rms_norm(x, eps) @ np.asarray(w, np.float64).T


def swiglu(x, w_gate, w_up) -> np.ndarray:
    """silu(x @ W_gate) * (x @ W_up) (reference mlx/kernels/standard/swiglu.py:9-10)."""
    x = np.asarray(x, np.float64)
    return silu(x @ np.asarray(w_gate, np.float64)) * (x @ np.asarray(w_up, np.float64))


def rope_embedding(x, base: float = 10000.0) -> np.ndarray:
    """Rows of x (S, D) rotated at positions 0..S-1 with omega_i = 1 / base^(2i/D)
    (reference mlx/kernels/standard/rope_embedding.py:15-32)."""
    x = np.asarray(x, np.float64)
    return rope_interleaved(x, np.arange(x.shape[0], dtype=np.float64), base)


def llama_attention(x, w_qkv, w_o, *, n_heads, n_kv_heads, base=10000.0):
    """GQA attention with RoPE, no cache, no mask, no norm or residual
    (reference mlx/kernels/standard/llama_attention.py:30-58): qkv = x W_qkv,
    q and k rotated at positions 0..S-1, query head h reads kv head h // G,
    softmax over all S keys, heads concatenated and projected by W_o."""
    x = np.asarray(x, np.float64)
    s_len, d = x.shape
    dh = d // n_heads
    g = n_heads // n_kv_heads
    qkv = x @ np.asarray(w_qkv, np.float64)
    pos = np.arange(s_len, dtype=np.float64)
    out = np.empty((s_len, d))
    for h in range(n_heads):
        kvh = h // g
        q = rope_interleaved(qkv[:, h * dh:(h + 1) * dh], pos, base)
        k = rope_interleaved(qkv[:, d + kvh * dh:d + (kvh + 1) * dh], pos, base)
        v = qkv[:, d + (n_kv_heads + kvh) * dh:d + (n_kv_heads + kvh + 1) * dh]
        out[:, h * dh:(h + 1) * dh] = softmax(q @ k.T / np.sqrt(dh), axis=-1) @ v
    return out @ np.asarray(w_o, np.float64)

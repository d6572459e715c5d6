"""Kernel registry (full set): whole-model blocks.

Same layout as reference mlx/kernels/full/registry.py (see the common
registry's docstring for the optional keys).  Outputs beyond the first sit at
bindings len(input_shapes)+1, +2, ... (`extra_outputs`), then the scalars.

This file is exec'd on its own by tools and tests, so it imports nothing.
"""

REGISTRY = {}

# ---- LLaMA decoder layer, one decode step (bf16) -----------------------------
# Hidden 4096, 32 query heads / 8 KV heads, head_dim 128, SwiGLU FFN 14336,
# RMSNorm eps 1e-5 (no gain, as reference llama_decoder_layer.py:48-50), RoPE
# theta 500000 (interleaved pairs, reference :52-64).  Batch 16; each sequence
# has 2048 cached positions (keys stored already rotated) and the new token at
# position 2048 attends to all 2049.  Weights normal(0, 0.02), x and caches
# normal(0, 1), all bf16.  Outputs: y [B, D], and the new token's rotated key
# and value [B, Hkv, Dh] for the caller to append.
_B, _D, _H, _HKV, _DH, _FF, _L = 16, 4096, 32, 8, 128, 14336, 2048
_QKV = _D + 2 * _HKV * _DH
_W = _D * _QKV + _D * _D + _D * 2 * _FF + _FF * _D
REGISTRY["llama_decoder_step"] = dict(
    metal_function="llama_decoder_step_bf16",
    threadgroup=(256, 1, 1),
    input_bindings=(0, 1, 2, 3, 4, 5, 6),
    input_shapes=[(_B, _D), (_D, _QKV), (_D, _D), (_D, 2 * _FF), (_FF, _D),
                  (_B, _HKV, _L, _DH), (_B, _HKV, _L, _DH)],
    output_shape=(_B, _D),
    extra_outputs=[dict(shape=(_B, _HKV, _DH), dtype="bf16"),
                   dict(shape=(_B, _HKV, _DH), dtype="bf16")],
    rtol=2e-2, atol=2e-2,
    grid=(1024 * 256, 1, 1),
    scalars=[dict(binding=10, dtype="u32", value=_B),
             dict(binding=11, dtype="u32", value=_D),
             dict(binding=12, dtype="u32", value=_H),
             dict(binding=13, dtype="u32", value=_HKV),
             dict(binding=14, dtype="u32", value=_FF),
             dict(binding=15, dtype="u32", value=_L),
             dict(binding=16, dtype="f32", value=500000.0),
             dict(binding=17, dtype="f32", value=1e-5)],
    # GEMMs 2*B*W, plus q.k and p.v over L+1 positions for every query head.
    flops=2 * _B * _W + 2 * 2 * _B * _H * (_L + 1) * _DH,
    # Weights once, KV cache read once, new k/v written, x read and y written.
    bytes=2 * _W + 2 * 2 * _B * _HKV * _L * _DH + 2 * 2 * _B * _HKV * _DH + 2 * 2 * _B * _D,
    input_dtypes=["bf16"] * 7,
    input_init=[("normal", 0.0, 1.0)] + [("normal", 0.0, 0.02)] * 4
               + [("normal", 0.0, 1.0)] * 2,
    output_dtype="bf16",
    compute_dtype="bf16",
    model_kwargs=dict(B=_B, D=_D, H=_H, H_kv=_HKV, FF=_FF, L=_L, base=500000.0, eps=1e-5),
    cpu_iters=3,
)

# ---- LLaMA decoder layer, prefill, the reference's own shape (fp32) ------------
# S 64 tokens at positions 0..63, D 128, 4 query heads / 2 KV heads (Dh 32),
# SwiGLU FFN 256, RoPE base 10000, RMSNorm eps 1e-5, full (non-causal)
# attention; all inputs normal(0, 1) (reference registry.py:87-104).
REGISTRY["llama_decoder_layer"] = dict(
    metal_function="llama_decoder_layer_f32",
    threadgroup=(256, 1, 1),
    input_bindings=(0, 1, 2, 3, 4),
    input_shapes=[(64, 128), (128, 128 + 2 * 2 * 32), (128, 128), (128, 2 * 256), (256, 128)],
    output_shape=(64, 128),
    rtol=1e-2, atol=1e-2,
    grid=(1024, 1, 1),
    scalars=[dict(binding=6, dtype="u32", value=64),
             dict(binding=7, dtype="u32", value=128),
             dict(binding=8, dtype="u32", value=4),
             dict(binding=9, dtype="u32", value=2),
             dict(binding=10, dtype="u32", value=256),
             dict(binding=11, dtype="f32", value=10000.0),
             dict(binding=12, dtype="f32", value=1e-5)],
    flops=64 * (128 * 256 * 2 + 64 * 128 * 2 + 128 * 128 * 2 + 128 * 512 * 2 + 256 * 128 * 2),
    bytes=4 * (64 * 128 * 3 + 128 * 256 + 128 * 128 + 128 * 512 + 256 * 128),
    compute_dtype="f32",
    model_kwargs=dict(S=64, D=128, H=4, H_kv=2, FF=256, base=10000.0, eps=1e-5),
)

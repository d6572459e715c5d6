"""Kernel registry (standard set): fused kernels, 2+ ops in one dispatch.

Same layout and keys as reference mlx/kernels/standard/registry.py (see the
common registry's docstring for the optional keys).  The entries here are the
LLaMA decoder's sub-ops at the reference's own shapes and tolerances; inputs
are normal(0, 1), as the reference's mx.random.normal
(mlx/scripts/mlx_helpers.py:241-251).

This file is exec'd on its own by tools and tests, so it imports nothing.
"""

REGISTRY = {}

# y = RMSNorm(x + residual), rows of 1024 (reference registry.py:280-292).
REGISTRY["fused_add_rms_norm"] = dict(
    metal_function="fused_add_rms_norm_f32",
    threadgroup=(1024, 1, 1),
    input_bindings=(0, 1),
    input_shapes=[(1024, 1024), (1024, 1024)],
    output_shape=(1024, 1024),
    rtol=1e-3, atol=1e-3,
    grid=(1024, 1024, 1),
    scalars=[dict(binding=3, dtype="u32", value=1024),
             dict(binding=4, dtype="f32", value=1e-5)],
    flops=1024 * 1024 * 6,
    bytes=4 * 1024 * 1024 * 3,
    model_kwargs=dict(dim=1024, eps=1e-5),
)

# y = rms_norm(x) @ W^T, W [out][in] (reference registry.py:26-42).
REGISTRY["rms_norm_linear"] = dict(
    metal_function="rms_norm_linear_f32",
    threadgroup=(512, 1, 1),
    input_bindings=(0, 1),
    input_shapes=[(1024, 1024), (1024, 1024)],
    output_shape=(1024, 1024),
    rtol=1e-3, atol=1e-3,
    grid=((1024 // 64) * 512, 1024 // 64, 1),
    scalars=[dict(binding=3, dtype="u32", value=1024),
             dict(binding=4, dtype="u32", value=1024),
             dict(binding=5, dtype="u32", value=1024),
             dict(binding=6, dtype="f32", value=1e-5)],
    flops=1024 * 1024 * 1024 * 2 + 1024 * 1024 * 5,
    bytes=1024 * 1024 * 4 * 3,
    compute_dtype="f32",
    model_kwargs=dict(dim=1024, out_dim=1024, eps=1e-5),
)

# RoPE over (S, D) with position = row, omega_i = 1 / 10000^(2i/D)
# (reference registry.py:103-117).
REGISTRY["rope_embedding"] = dict(
    metal_function="rope_embedding_f32",
    threadgroup=(256, 1, 1),
    input_bindings=(0,),
    input_shapes=[(128, 64)],
    output_shape=(128, 64),
    rtol=1e-4, atol=1e-5,
    grid=(((128 * 32) + 255) // 256 * 256, 1, 1),
    scalars=[dict(binding=2, dtype="u32", value=128),
             dict(binding=3, dtype="u32", value=64),
             dict(binding=4, dtype="f32", value=10000.0)],
    flops=128 * 32 * 6,
    bytes=128 * 64 * 4 * 2,
    model_kwargs=dict(base=10000.0),
)

# silu(x @ W_gate) * (x @ W_up), 256^3 (reference registry.py:119-133).
REGISTRY["swiglu"] = dict(
    metal_function="swiglu_f32",
    threadgroup=(512, 1, 1),
    input_bindings=(0, 1, 2),
    input_shapes=[(256, 256), (256, 256), (256, 256)],
    output_shape=(256, 256),
    rtol=1e-3, atol=1e-3,
    grid=(((256 * 256) + 255) // 256 * 256, 1, 1),
    scalars=[dict(binding=4, dtype="u32", value=256),
             dict(binding=5, dtype="u32", value=256),
             dict(binding=6, dtype="u32", value=256)],
    flops=256 * 256 * 256 * 4 + 256 * 256 * 5,
    bytes=4 * (256 * 256 * 3 + 256 * 256),
    compute_dtype="f32",
)

# x @ W_qkv -> (Q | K | V), 128 x 512 @ 512 x 192 (reference registry.py:324-337).
REGISTRY["fused_qkv_projection"] = dict(
    metal_function="fused_qkv_projection_f32",
    threadgroup=(512, 1, 1),
    input_bindings=(0, 1),
    input_shapes=[(128, 512), (512, 192)],
    output_shape=(128, 192),
    rtol=1e-3, atol=1e-3,
    grid=(((128 * 192) + 255) // 256 * 256, 1, 1),
    scalars=[dict(binding=3, dtype="u32", value=128),
             dict(binding=4, dtype="u32", value=192),
             dict(binding=5, dtype="u32", value=512)],
    flops=2 * 128 * 192 * 512,
    bytes=4 * (128 * 512 + 512 * 192 + 128 * 192),
    compute_dtype="f32",
)

# GQA attention with RoPE, no cache, no mask: S 64, D 128, 4 query heads,
# 2 kv heads (reference registry.py:398-413).
REGISTRY["llama_attention"] = dict(
    metal_function="llama_attention_f32",
    threadgroup=(256, 1, 1),
    input_bindings=(0, 1, 2),
    input_shapes=[(64, 128), (128, 128 + 2 * 2 * 32), (128, 128)],
    output_shape=(64, 128),
    rtol=1e-2, atol=1e-2,
    grid=(1024, 1, 1),
    scalars=[dict(binding=4, dtype="u32", value=64),
             dict(binding=5, dtype="u32", value=128),
             dict(binding=6, dtype="u32", value=4),
             dict(binding=7, dtype="u32", value=2),
             dict(binding=8, dtype="f32", value=10000.0)],
    flops=64 * (128 * (128 + 128) * 2 + 64 * 128 * 2 + 128 * 128 * 2),
    bytes=4 * (64 * 128 * 2 + 128 * 256 + 128 * 128),
    compute_dtype="f32",
    model_kwargs=dict(S=64, D=128, H=4, H_kv=2, base=10000.0),
)

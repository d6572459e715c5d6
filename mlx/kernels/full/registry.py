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
def _decode_step(name, B, D, H, HKV, DH, FF, L):
    QD = H * DH                     # attention width: D for a whole layer
    QKV = QD + 2 * HKV * DH
    W = D * QKV + QD * D + D * 2 * FF + FF * D
    REGISTRY[name] = dict(
        metal_function="llama_decoder_step_bf16",
        threadgroup=(256, 1, 1),
        input_bindings=(0, 1, 2, 3, 4, 5, 6),
        input_shapes=[(B, D), (D, QKV), (QD, D), (D, 2 * FF), (FF, D),
                      (B, HKV, L, DH), (B, HKV, L, DH)],
        output_shape=(B, D),
        extra_outputs=[dict(shape=(B, HKV, DH), dtype="bf16"),
                       dict(shape=(B, HKV, DH), dtype="bf16")],
        rtol=2e-2, atol=2e-2,
        grid=(1024 * 256, 1, 1),
        scalars=[dict(binding=10, dtype="u32", value=B),
                 dict(binding=11, dtype="u32", value=D),
                 dict(binding=12, dtype="u32", value=H),
                 dict(binding=13, dtype="u32", value=HKV),
                 dict(binding=14, dtype="u32", value=FF),
                 dict(binding=15, dtype="u32", value=L),
                 dict(binding=16, dtype="f32", value=500000.0),
                 dict(binding=17, dtype="f32", value=1e-5)],
        # GEMMs 2*B*W, plus q.k and p.v over L+1 positions for every query head.
        flops=2 * B * W + 2 * 2 * B * H * (L + 1) * DH,
        # Weights once, KV cache read once, new k/v written, x read and y written.
        bytes=2 * W + 2 * 2 * B * HKV * L * DH + 2 * 2 * B * HKV * DH + 2 * 2 * B * D,
        input_dtypes=["bf16"] * 7,
        input_init=[("normal", 0.0, 1.0)] + [("normal", 0.0, 0.02)] * 4
                   + [("normal", 0.0, 1.0)] * 2,
        output_dtype="bf16",
        compute_dtype="bf16",
        model_kwargs=dict(B=B, D=D, H=H, H_kv=HKV, FF=FF, L=L, base=500000.0, eps=1e-5,
                          D_head=DH),
        cpu_iters=3,
    )


_decode_step("llama_decoder_step", 16, 4096, 32, 8, 128, 14336, 2048)

# One GPU's share of the same step under 8-way tensor parallelism: 4 of the 32
# query heads and 1 of the 8 KV heads (W_qkv 4096 x 768), the matching 512
# rows of W_o, 1792 of the 14336 gate and up columns (W_gu 4096 x 3584) and
# rows of W_down (1792 x 4096), the KV cache of its head [16, 1, 2048, 128].
# It is a cost proxy for one shard's work, not a usable shard: the step adds
# the full residual and normalises its own partial x1, so the shards' outputs
# do not all-reduce to the layer's (a real shard splits the step at W_o and
# all-reduces between the halves).
_decode_step("llama_decoder_step_tp8", 16, 4096, 4, 1, 128, 1792, 2048)

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

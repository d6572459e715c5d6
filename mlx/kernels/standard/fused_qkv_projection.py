"""Fused QKV projection x @ W_qkv -> (Q | K | V) (spec of reference
mlx/kernels/standard/fused_qkv_projection.py:5-13), run on the host CPU in fp32."""
import torch


class Model(torch.nn.Module):
    """Fused QKV projection: x (S, D_in) @ W_qkv (D_in, 3 D_head)."""

    def forward(self, x: torch.Tensor, w_qkv: torch.Tensor) -> torch.Tensor:
        return x @ w_qkv

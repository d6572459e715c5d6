"""Rotary position embedding over (S, D) (spec of reference
mlx/kernels/standard/rope_embedding.py:5-32): for position p = row and pair
(2i, 2i+1), rotate by p * omega_i with omega_i = 1 / base^(2i / D).  Run on
the host CPU in fp32."""
import torch


class Model(torch.nn.Module):
    """RoPE: rotary position embedding of x (S, D), D even."""

    def __init__(self, base: float = 10000.0):
        super().__init__()
        self.base = base

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        S, D = x.shape
        half = D // 2
        idx = torch.arange(half, dtype=torch.float32)
        omega = 1.0 / (self.base ** (2.0 * idx / D))
        pos = torch.arange(S, dtype=torch.float32)
        ang = pos[:, None] * omega[None, :]
        cos, sin = torch.cos(ang), torch.sin(ang)
        x0, x1 = x[:, 0::2], x[:, 1::2]
        return torch.stack([x0 * cos - x1 * sin, x0 * sin + x1 * cos], dim=-1).reshape(S, D)

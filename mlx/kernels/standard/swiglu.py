"""SwiGLU, silu(x @ W_gate) * (x @ W_up) (spec of reference
mlx/kernels/standard/swiglu.py:5-10), run on the host CPU in fp32."""
import torch
import torch.nn.functional as F


class Model(torch.nn.Module):
    """SwiGLU: silu(x @ W_gate) * (x @ W_up)."""

    def forward(self, x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
        return F.silu(x @ w_gate) * (x @ w_up)

"""RMSNorm + linear, y = rms_norm(x) @ W^T (spec of reference
mlx/kernels/standard/rms_norm_linear.py:5-14: the forward normalises with eps
1e-5 and no gain, then multiplies by the transposed weight), run on the host
CPU in fp32."""
import torch


class Model(torch.nn.Module):
    """RMSNorm + Linear: y = rms_norm(x) @ W^T."""

    def __init__(self, dim=1024, out_dim=1024, eps=1e-5):
        super().__init__()
        self.eps = eps

    def forward(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        n = x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + self.eps)
        return n @ w.t()

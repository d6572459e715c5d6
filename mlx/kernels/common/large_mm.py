"""Large bf16 GEMM: C = A @ B with bf16 operands and fp32 accumulation.

The reference has no bf16 kernel; this is its matmul spec (reference
mlx/kernels/common/sqr_mm.py:10-11) at bf16.  The spec value is the
fp32-accumulated product of the bf16 operands, kept in fp32 (the kernel's bf16
output is compared against it with rtol 1e-2)."""
import torch


class Model(torch.nn.Module):
    """bf16 matrix multiplication with fp32 accumulation: C = A @ B."""

    def forward(self, A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
        return torch.matmul(A.float(), B.float())

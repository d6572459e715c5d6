"""Large bf16 GEMM: C = A @ B with bf16 operands, fp32 accumulation and a bf16
result.

The reference has no bf16 kernel; this is its matmul spec (reference
mlx/kernels/common/sqr_mm.py:10-11) at bf16, with mx.matmul's semantics on
bf16 arrays: the products are summed in fp32 and the result is rounded to
bf16 once.  torch's CPU matmul of bf16 tensors does the same (fp32
accumulation inside), so the spec runs at the workload's own precision."""
import torch


class Model(torch.nn.Module):
    """bf16 matrix multiplication with fp32 accumulation: C = A @ B."""

    def forward(self, A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
        return torch.matmul(A, B)

"""LLaMA-style grouped-query attention with RoPE, no cache and no mask (spec
of reference mlx/kernels/standard/llama_attention.py:5-58), run on the host CPU
in fp32: qkv = x @ W_qkv; q, k rotated by their positions (interleaved pairs,
omega_i = base^(-2i/Dh)); query head h reads kv head h // G; softmax over all
S keys; output heads concatenated and projected by W_o.  Computed in float64:
with the reference's normal(0, 1) weights the activations reach the hundreds,
where fp32 rounding alone approaches the registry's atol."""
import math

import torch


class Model(torch.nn.Module):
    """Grouped-query attention with RoPE: (S, D) -> (S, D)."""

    def __init__(self, S=64, D=128, H=4, H_kv=2, base=10000.0):
        super().__init__()
        self.S, self.D, self.H, self.H_kv, self.base = S, D, H, H_kv, base
        self.D_head = D // H
        self.G = H // H_kv

    def _rope(self, t: torch.Tensor) -> torch.Tensor:
        heads, S, Dh = t.shape
        idx = torch.arange(Dh // 2, dtype=torch.float64)
        omega = 1.0 / (self.base ** (2.0 * idx / Dh))
        ang = torch.arange(S, dtype=torch.float64)[:, None] * omega[None, :]
        c, s = torch.cos(ang), torch.sin(ang)
        t0, t1 = t[..., 0::2], t[..., 1::2]
        return torch.stack([t0 * c - t1 * s, t0 * s + t1 * c], dim=-1).reshape(heads, S, Dh)

    def forward(self, x, W_qkv, W_o):
        out_dtype = x.dtype
        x, W_qkv, W_o = x.double(), W_qkv.double(), W_o.double()
        S, D, H, H_kv, Dh = self.S, self.D, self.H, self.H_kv, self.D_head
        qkv = x @ W_qkv
        q = qkv[:, :D].reshape(S, H, Dh).transpose(0, 1)
        k = qkv[:, D:D + H_kv * Dh].reshape(S, H_kv, Dh).transpose(0, 1)
        v = qkv[:, D + H_kv * Dh:].reshape(S, H_kv, Dh).transpose(0, 1)
        q, k = self._rope(q), self._rope(k)
        k = k.repeat_interleave(self.G, dim=0)
        v = v.repeat_interleave(self.G, dim=0)
        scores = (q @ k.transpose(1, 2)) / math.sqrt(Dh)
        out = torch.softmax(scores, dim=-1) @ v
        return (out.transpose(0, 1).reshape(S, D) @ W_o).to(out_dtype)

"""The compression-gate producer, as the reference's ``CompressionGate``
(common.py:288-328): ``Linear(dim, dim)`` on the DiT hidden states, returned as
the per-head view ``[B, H, S, D]`` of its ``[B, S, dim]`` output.

On MI355X the GEMM is a plain library GEMM (hipBLASLt through ``F.linear``),
and the view is never materialised: ``mi355x_vsa`` recognises a gate that is
the per-head transpose of a contiguous ``[B, S, H, D]`` tensor, reads it in
place in the combine epilogue of the fine forward, and writes the gate
gradient in the same token-major layout, so neither direction pays a
transpose copy of a full ``[B, H, S, D]`` tensor.
"""

from __future__ import annotations

from torch import Tensor, nn


class CompressionGate(nn.Module):
    """``to_gate_compress``: hidden states ``[batch, seq_len, dim]`` ->
    per-head gate ``[batch, heads, seq_len, dim / heads]`` (a view)."""

    def __init__(self, dim: int, num_heads: int, bias: bool = True) -> None:
        super().__init__()
        if dim % num_heads:
            raise ValueError(f"dim={dim} must be divisible by num_heads={num_heads}")
        self.num_heads = num_heads
        self.to_gate_compress = nn.Linear(dim, dim, bias=bias)

    def forward(self, hidden_states: Tensor) -> Tensor:
        if hidden_states.ndim != 3:
            raise ValueError("hidden_states must have shape [batch, seq_len, dim]")
        b, s, _ = hidden_states.shape
        gate = self.to_gate_compress(hidden_states)          # [B, S, dim], contiguous
        return gate.view(b, s, self.num_heads, -1).transpose(1, 2)

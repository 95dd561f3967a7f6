"""RoPE tables and the unfused rotate-half semantics (caller side of the op).

``RotaryEmbedding`` builds the fp32 cos/sin tables the decoder passes to
``fused_qkv_rope`` after casting them to bf16 (reference
mini_qwen/model/layers/rope.py:6-21; the caller casts at model/qwen3.py:140-142
for prefill and indexes ``cos_cached[positions]`` at :163-165 for decode).
Layout: ``emb = cat([freqs, freqs])`` so both halves of a row carry the same
angles; the kernels still read both halves, as the reference kernel does.
"""
from __future__ import annotations

from typing import Tuple

import torch
import torch.nn as nn


def rope_tables(head_dim: int, max_seq_len: int, theta: float = 1.0e6, device=None):
    """fp32 ``(cos, sin)``, each ``[max_seq_len, head_dim]``.

    Angle of position p, pair i: ``p * theta ** (-2i / head_dim)`` computed as
    ``p * (1 / theta ** (2i / head_dim))`` in fp32, duplicated over both halves
    -- the same fp32 operations as the reference (rope.py:9, :14-17), so the
    tables are bitwise equal to its buffers on the same torch build.
    """
    if head_dim % 2 != 0:
        raise ValueError("head_dim must be even")
    exps = torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim
    inv_freq = 1.0 / (theta ** exps)
    pos = torch.arange(max_seq_len, dtype=torch.float32, device=device)
    angles = torch.outer(pos, inv_freq).repeat(1, 2)
    return angles.cos(), angles.sin()


class RotaryEmbedding(nn.Module):
    """Holds ``cos_cached`` / ``sin_cached`` for ``theta`` (default 1e6, Qwen3)."""

    def __init__(self, head_dim: int, max_seq_len: int = 40960, theta: float = 1000000.0,
                 device=None):
        super().__init__()
        cos, sin = rope_tables(head_dim, max_seq_len, theta, device)
        self.register_buffer("cos_cached", cos, persistent=False)
        self.register_buffer("sin_cached", sin, persistent=False)

    def forward(self, seq_len: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Prefill tables: the first ``seq_len`` rows (fp32)."""
        return self.cos_cached[:seq_len], self.sin_cached[:seq_len]

    def rows(self, positions: torch.Tensor, dtype=torch.bfloat16) -> Tuple[torch.Tensor, torch.Tensor]:
        """Per-token rows ``[T, D]`` for decode (model/qwen3.py:163-165)."""
        idx = positions.to(device=self.cos_cached.device, dtype=torch.long)
        return self.cos_cached[idx].to(dtype), self.sin_cached[idx].to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """``[x1, x2] -> [-x2, x1]`` over the last axis (rope.py:24-28)."""
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


def apply_rotary_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """Unfused RoPE for ``q, k [B, S, H, D]`` and ``cos, sin [S, D]`` (rope.py:31-45)."""
    c = cos.unsqueeze(0).unsqueeze(2)
    s = sin.unsqueeze(0).unsqueeze(2)
    return q * c + rotate_half(q) * s, k * c + rotate_half(k) * s

"""Caller-side layer: the attn-bench multi-head self-attention wrapper.

Mirrors ``attn-bench/src/layers/attention/morpho_attention.py:9-41``: the same
class name, constructor (``dim, num_heads, dropout=0.0, *, cube_m=64,
scale=None, causal=False, **_``), attributes (``name``, ``num_heads``,
``head_dim``, ``cube_m``, ``scale``, ``causal``, ``attn``, ``proj``,
``dropout``) and forward contract: ``forward(x, k, v, attn_bias=None)`` runs
morpho attention on ``x`` in fp16 (``k``, ``v`` and ``attn_bias`` are accepted
and ignored, as there), casts back to the input dtype, applies the output
projection and dropout, and returns ``(out, None)``.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import nn

from .autograd import MorphoAttention


class MultiHeadSelfAttention(nn.Module):
    """Multi-head self-attention layer built on :class:`MorphoAttention`.

    :param dim: model dimension (divisible by ``num_heads``).
    :param num_heads: number of heads.
    :param dropout: dropout probability after the output projection.
    :param cube_m: hypercube width per head (16, 32 or 64).
    :param scale: softmax temperature; ``cube_m ** -0.5`` when ``None``.
    :param causal: causal masking.
    """

    HEAD_DIM = 64
    CUBE_M = 64

    def __init__(self, dim: int, num_heads: int, dropout: float = 0.0, *, cube_m: int = CUBE_M,
                 scale: float | None = None, causal: bool = False, **_: Any) -> None:
        super().__init__()
        self.name = "morpho_attention"
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.cube_m = cube_m
        self.scale = scale if scale is not None else cube_m ** -0.5
        self.causal = causal
        self.attn = MorphoAttention(dim, num_heads, cube_m, scale=self.scale, causal=causal)
        self.proj = nn.Linear(dim, dim)
        self.dropout = nn.Dropout(dropout)

    def forward(self, x: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                attn_bias: torch.Tensor | None = None) -> tuple[torch.Tensor, None]:
        orig_dtype = x.dtype
        out = self.attn(x.to(torch.float16)).to(orig_dtype)
        out = self.proj(out)
        return self.dropout(out), None

"""Soft tropical aggregation on the MI355X kernels.

The reference defines soft max-plus / min-plus log-sum-exp accumulators in
``packages/morphottention/csrc/cuda/morfology/soft_morph.cuh:10-77``
(``morph_accumulate``, ``lse_merge``, ``lse_finalize``, ``morph_weight``,
``morph_dtau_term``) but never wires them to a kernel, op or module. Here they
aggregate the values with the morpho scores in place of the softmax-weighted
sum:

    out_ic = sgn * tau * ln sum_j exp(sgn * (s_ij + V_jc) / tau)

with ``s_ij`` the scores of ``MorphoAttention`` (natural-log units, including
``scale``), ``sgn = +1`` the soft dilation (max-plus) and ``sgn = -1`` the
soft erosion (min-plus). As ``tau -> 0`` the output tends to
``max_j (s_ij + V_jc)`` (or the min). ``tau`` is a learnable float32
parameter; its gradient is ``morph_dtau_term`` summed over every output.
"""

from __future__ import annotations

import torch
from torch import nn

from . import capi
from ._ops import add_op_namespace_prefix, ops
from .autograd import variant_bits


@torch.library.register_fake(add_op_namespace_prefix("soft_forward"))
def _soft_forward_fake(X, W_phi, gate_q, gate_k, W_V, tau, H, cube_m, scale, causal, sgn, variant=0):
    B, N, D = X.shape
    ws = X.new_empty((capi.soft_forward_workspace_size(B, N, D, H, cube_m),), dtype=torch.uint8)
    return [torch.empty_like(X), X.new_empty((B * H, N, D // H), dtype=torch.float32), ws]


@torch.library.register_fake(add_op_namespace_prefix("soft_backward"))
def _soft_backward_fake(grad_out, X, W_phi, gate_q, gate_k, W_V, tau, zb, workspace, H, cube_m, scale, causal, sgn,
                        variant=0):
    return [torch.empty_like(X), torch.empty_like(W_phi), torch.empty_like(gate_q), torch.empty_like(gate_k),
            torch.empty_like(W_V), torch.empty_like(tau)]


class SoftMorphAttentionFunction(torch.autograd.Function):
    """Autograd bridge of ``soft_forward`` / ``soft_backward``: gradients for
    ``x``, ``W_phi``, ``gate_q``, ``gate_k``, ``W_V`` and ``tau``."""

    @staticmethod
    def forward(ctx, x, W_phi, gate_q, gate_k, W_V, tau, H, cube_m, scale, causal, sgn, variant=0):
        if not x.is_cuda:
            raise ValueError("SoftMorphAttention expects a CUDA tensor")
        x = x.contiguous()
        out, zb, ws = ops.soft_forward(x, W_phi, gate_q, gate_k, W_V, tau, H, cube_m, scale, causal, sgn, variant)
        ctx.save_for_backward(x, W_phi, gate_q, gate_k, W_V, tau, zb, ws)
        ctx.args = (H, cube_m, scale, causal, sgn, variant)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, W_phi, gate_q, gate_k, W_V, tau, zb, ws = ctx.saved_tensors
        grads = ops.soft_backward(grad_out.contiguous(), x, W_phi, gate_q, gate_k, W_V, tau, zb, ws, *ctx.args)
        return (*grads, None, None, None, None, None, None)


# Mode bit of the soft ops: always run the element-wise kernels instead of the
# product form on MFMA (which falls back to them by itself where its
# precision guarantee does not hold).
SOFT_EXACT = 16


def soft_morph_attention(x, W_phi, gate_q, gate_k, W_V, tau, num_heads: int, cube_m: int, *, scale: float = 1.0,
                         causal: bool = False, erosion: bool = False, projection: str = "sigmoid",
                         mask_diag: bool = False, exact: bool = False) -> torch.Tensor:
    """Soft tropical aggregation with autograd support.

    :param tau: float32 CUDA tensor with one element, the temperature (> 0).
    :param erosion: soft min-plus (``sgn = -1``) instead of soft max-plus.
    :param exact: always use the element-wise kernels (one exp2 per query,
        key and value column) instead of the product form on MFMA.
    """
    variant = variant_bits(projection, mask_diag) | (SOFT_EXACT if exact else 0)
    return SoftMorphAttentionFunction.apply(x, W_phi, gate_q, gate_k, W_V, tau, num_heads, cube_m, scale, causal,
                                            -1 if erosion else 1, variant)


class SoftMorphAttention(nn.Module):
    """Morpho scores with soft tropical value aggregation.

    Parameters and their default initialisation are those of
    ``MorphoAttention`` (``W_phi``, ``gate_q``, ``gate_k``, ``W_V``), plus
    ``tau``: a float32 parameter of one element (a buffer when
    ``learn_tau=False``).
    """

    def __init__(self, dim: int, num_heads: int, cube_m: int, *, scale: float = 1.0, causal: bool = False,
                 tau: float = 1.0, erosion: bool = False, learn_tau: bool = True,
                 dtype: torch.dtype = torch.float16, device: torch.device | str | None = None,
                 projection: str = "sigmoid", mask_diag: bool = False) -> None:
        super().__init__()
        if dim % num_heads != 0:
            raise ValueError(f"dim ({dim}) must be divisible by num_heads ({num_heads})")
        if not tau > 0:
            raise ValueError(f"tau must be positive (got {tau})")
        self.variant = variant_bits(projection, mask_diag)
        self.dim = dim
        self.num_heads = num_heads
        self.cube_m = cube_m
        self.scale = scale
        self.causal = causal
        self.sgn = -1 if erosion else 1
        head_dim_v = dim // num_heads
        self.W_phi = nn.Parameter(torch.empty(dim, num_heads * cube_m, dtype=dtype, device=device))
        self.gate_q = nn.Parameter(torch.empty(num_heads, cube_m, dtype=dtype, device=device))
        self.gate_k = nn.Parameter(torch.empty(num_heads, cube_m, dtype=dtype, device=device))
        self.W_V = nn.Parameter(torch.empty(dim, num_heads * head_dim_v, dtype=dtype, device=device))
        t = torch.full((1,), float(tau), dtype=torch.float32, device=device)
        if learn_tau:
            self.tau = nn.Parameter(t)
        else:
            self.register_buffer("tau", t)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        std = self.dim ** -0.5
        with torch.no_grad():
            for w in (self.W_phi, self.W_V):
                w.copy_(torch.empty(w.shape, dtype=torch.float32, device=w.device).normal_(0.0, std))
            self.gate_q.fill_(1.0)
            self.gate_k.fill_(1.0)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return SoftMorphAttentionFunction.apply(x, self.W_phi, self.gate_q, self.gate_k, self.W_V, self.tau,
                                                self.num_heads, self.cube_m, self.scale, self.causal, self.sgn,
                                                self.variant)

"""Autograd bridge and nn.Module around the MI355X morpho-attention kernels.

Drop-in for ``packages/morphottention/torch-ext/morphottention/autograd.py``:
``MorphoAttention`` (``:91-140``), ``morpho_attention`` (``:143-162``) and
``MorphoAttentionFunction`` (``:34-88``) keep their names, signatures, parameter
names, default initialisation and errors. Differences, all deliberate:

* ``causal`` takes effect (the reference's kernels ignore it);
* the backward returns the complete gradient (the reference drops the
  query-side code terms);
* the Function calls ``forward_train`` / ``backward_train``, which carry the
  forward's projection workspace to the backward instead of recomputing it;
  the reference ops ``forward`` / ``backward`` remain available with their
  original schemas (``backward`` then recomputes the projection);
* the op ``forward`` is itself differentiable (``torch.library.register_autograd``,
  backward through the reference-schema ``backward`` op), and every op has a
  fake, so ``torch.compile`` traces the module without graph breaks.
"""

from __future__ import annotations

import torch
from torch import nn

from . import capi
from ._ops import add_op_namespace_prefix, ops


@torch.library.register_fake(add_op_namespace_prefix("forward"))
def _morpho_forward_fake(X, W_phi, gate_q, gate_k, W_V, H, cube_m, scale, causal):
    B, N, _D = X.shape
    out = torch.empty_like(X)
    lse = X.new_empty((B * H, N), dtype=torch.float32)
    return [out, lse]


@torch.library.register_fake(add_op_namespace_prefix("forward_train"))
def _morpho_forward_train_fake(X, W_phi, gate_q, gate_k, W_V, H, cube_m, scale, causal, variant=0):
    B, N, D = X.shape
    ws = X.new_empty((capi.forward_workspace_size(B, N, D, H, cube_m),), dtype=torch.uint8)
    return [torch.empty_like(X), X.new_empty((B * H, N), dtype=torch.float32), ws]


def _grads_fake(X, W_phi, gate_q, gate_k, W_V):
    return [torch.empty_like(X), torch.empty_like(W_phi), torch.empty_like(gate_q), torch.empty_like(gate_k),
            torch.empty_like(W_V)]


@torch.library.register_fake(add_op_namespace_prefix("backward"))
def _morpho_backward_fake(grad_out, X, W_phi, gate_q, gate_k, W_V, out, lse, H, cube_m, scale, causal):
    return _grads_fake(X, W_phi, gate_q, gate_k, W_V)


@torch.library.register_fake(add_op_namespace_prefix("backward_train"))
def _morpho_backward_train_fake(grad_out, X, W_phi, gate_q, gate_k, W_V, out, lse, workspace, H, cube_m, scale,
                                causal, variant=0):
    return _grads_fake(X, W_phi, gate_q, gate_k, W_V)


# Autograd of the reference-schema op itself, so that
# torch.ops.morphottention.forward is differentiable without the Function
# (torch.compile / AOT autograd trace it through the fakes above). Its backward
# is the reference-schema ``backward`` op, which recomputes the projection; lse
# is treated as a non-differentiable statistic (its gradient is ignored).
def _forward_setup_context(ctx, inputs, output):
    x, W_phi, gate_q, gate_k, W_V, H, cube_m, scale, causal = inputs
    out, lse = output
    ctx.save_for_backward(x, W_phi, gate_q, gate_k, W_V, out, lse)
    ctx.meta = (H, cube_m, scale, causal)


def _forward_backward(ctx, grads):
    grad_out = grads[0]
    x, W_phi, gate_q, gate_k, W_V, out, lse = ctx.saved_tensors
    H, cube_m, scale, causal = ctx.meta
    if grad_out is None:
        grad_out = torch.zeros_like(out)
    dX, dW_phi, d_gate_q, d_gate_k, dW_V = ops.backward(grad_out.contiguous(), x, W_phi, gate_q, gate_k, W_V, out,
                                                        lse, H, cube_m, scale, causal)
    return dX, dW_phi, d_gate_q, d_gate_k, dW_V, None, None, None, None


torch.library.register_autograd(add_op_namespace_prefix("forward"), _forward_backward,
                                setup_context=_forward_setup_context)


# Variant bits of the *_train ops (the C ABI's morpho_mode without the causal
# bit): the reference's compile-time MASK_DIAG (declarations.cuh:79-82) and
# cube projections (cube.cuh:9-17), which it never wires to its API.
_MASK_DIAG = 2
_PROJECTIONS = {"sigmoid": 0, "hardtanh01": 4, "identity": 8}
# No reference counterpart: a backward whose gradients are the same bits on
# every run (the dq and row sums from per-key-block partials added in a fixed
# order instead of fp32 atomics; more workspace).
_DETERMINISTIC = 32


def variant_bits(projection: str = "sigmoid", mask_diag: bool = False, deterministic: bool = False) -> int:
    """Variant argument for ``forward_train`` / ``backward_train``."""
    if projection not in _PROJECTIONS:
        raise ValueError(f"projection must be one of {sorted(_PROJECTIONS)} (got {projection!r})")
    return _PROJECTIONS[projection] | (_MASK_DIAG if mask_diag else 0) | (_DETERMINISTIC if deterministic else 0)


class MorphoAttentionFunction(torch.autograd.Function):
    """Bridges the HIP attention kernels into autograd. The optional trailing
    ``variant`` (see :func:`variant_bits`) defaults to the reference's
    behaviour: sigmoid projection, diagonal kept."""

    @staticmethod
    def forward(ctx, x, W_phi, gate_q, gate_k, W_V, H, cube_m, scale, causal, variant=0):
        if not x.is_cuda:
            raise ValueError("MorphoAttention expects a CUDA tensor")
        x = x.contiguous()
        out, lse, ws = ops.forward_train(x, W_phi, gate_q, gate_k, W_V, H, cube_m, scale, causal, variant)
        ctx.save_for_backward(x, W_phi, gate_q, gate_k, W_V, out, lse, ws)
        ctx.H = H
        ctx.cube_m = cube_m
        ctx.scale = scale
        ctx.causal = causal
        ctx.variant = variant
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, W_phi, gate_q, gate_k, W_V, out, lse, ws = ctx.saved_tensors
        grad_out = grad_out.contiguous()
        dX, dW_phi, d_gate_q, d_gate_k, dW_V = ops.backward_train(
            grad_out, x, W_phi, gate_q, gate_k, W_V, out, lse, ws, ctx.H, ctx.cube_m, ctx.scale, ctx.causal,
            ctx.variant)
        return dX, dW_phi, d_gate_q, d_gate_k, dW_V, None, None, None, None, None


class MorphoAttention(nn.Module):
    """Morphological hypercube attention.

    :param dim: model dimension ``D`` (must be divisible by ``num_heads``).
    :param num_heads: number of attention heads ``H``.
    :param cube_m: hypercube width per head ``m`` (the score contraction dim);
        16, 32 or 64.
    :param scale: softmax temperature.
    :param causal: whether to apply causal masking.
    :param projection: cube projection ``"sigmoid"`` (the reference's
        default), ``"hardtanh01"`` or ``"identity"`` (the reference's unwired
        compile-time variants).
    :param mask_diag: drop each query's own key (the reference's unwired
        ``MASK_DIAG``).
    :param deterministic: bitwise run-to-run reproducible gradients (no
        reference counterpart; the backward needs more workspace).
    """

    def __init__(self, dim: int, num_heads: int, cube_m: int, *, scale: float = 1.0, causal: bool = False,
                 dtype: torch.dtype = torch.float16, device: torch.device | str | None = None,
                 projection: str = "sigmoid", mask_diag: bool = False, deterministic: bool = False) -> None:
        super().__init__()
        if dim % num_heads != 0:
            raise ValueError(f"dim ({dim}) must be divisible by num_heads ({num_heads})")
        self.variant = variant_bits(projection, mask_diag, deterministic)
        self.projection = projection
        self.mask_diag = mask_diag
        self.deterministic = deterministic
        self.dim = dim
        self.num_heads = num_heads
        self.cube_m = cube_m
        self.scale = scale
        self.causal = causal
        head_dim_v = dim // num_heads
        self.W_phi = nn.Parameter(torch.empty(dim, num_heads * cube_m, dtype=dtype, device=device))
        self.gate_q = nn.Parameter(torch.empty(num_heads, cube_m, dtype=dtype, device=device))
        self.gate_k = nn.Parameter(torch.empty(num_heads, cube_m, dtype=dtype, device=device))
        self.W_V = nn.Parameter(torch.empty(dim, num_heads * head_dim_v, dtype=dtype, device=device))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        std = self.dim ** -0.5
        with torch.no_grad():
            for w in (self.W_phi, self.W_V):
                w.copy_(torch.empty(w.shape, dtype=torch.float32, device=w.device).normal_(0.0, std))
            self.gate_q.fill_(1.0)
            self.gate_k.fill_(1.0)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return MorphoAttentionFunction.apply(x, self.W_phi, self.gate_q, self.gate_k, self.W_V, self.num_heads,
                                             self.cube_m, self.scale, self.causal, self.variant)


def morpho_attention(x, W_phi, gate_q, gate_k, W_V, num_heads: int, cube_m: int, *, scale: float = 1.0,
                     causal: bool = False, projection: str = "sigmoid", mask_diag: bool = False,
                     deterministic: bool = False) -> torch.Tensor:
    """Apply Morphottention attention with autograd support.

    :param x: input activations of shape (B, N, D) on a ROCm device.
    :param projection: ``"sigmoid"`` (default), ``"hardtanh01"`` or ``"identity"``.
    :param mask_diag: drop each query's own key.
    :param deterministic: bitwise run-to-run reproducible gradients.
    :returns: the attention output, differentiable w.r.t. ``x`` and the parameters.
    """
    return MorphoAttentionFunction.apply(x, W_phi, gate_q, gate_k, W_V, num_heads, cube_m, scale, causal,
                                         variant_bits(projection, mask_diag, deterministic))

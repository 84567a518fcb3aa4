"""Pins of the soft tropical aggregation oracle (no GPU).

The reference defines the accumulators in
``packages/morphottention/csrc/cuda/morfology/soft_morph.cuh:10-77`` but never
calls them, so it holds no tests or vectors for them. The oracle
``mo.soft_morph_ref`` (``out_ic = sgn tau ln sum_j exp(sgn (s_ij + V_jc) / tau)``)
is pinned here against a scalar restatement of the reference's own
accumulators and against what the mathematics fixes: the hard max-plus /
min-plus limit, the large-tau expansion with Hoeffding's bound, the
erosion-dilation duality, a single key, the partition of unity of the
weights, the tau-gradient identity and fp64 gradcheck.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import morpho_oracle as mo


def _inputs(B, N, D, H, m, seed=0, x_mult=1.0):
    g = torch.Generator().manual_seed(seed)
    x = x_mult * torch.randn(B, N, D, generator=g, dtype=torch.float64)
    W_phi = torch.randn(D, H * m, generator=g, dtype=torch.float64) * D ** -0.5
    W_V = torch.randn(D, D, generator=g, dtype=torch.float64) * D ** -0.5
    gq = 1.0 + 0.5 * torch.randn(H, m, generator=g, dtype=torch.float64)
    gk = 1.0 + 0.5 * torch.randn(H, m, generator=g, dtype=torch.float64)
    return x, W_phi, gq, gk, W_V


def _sv(x, W_phi, gq, gk, W_V, H, m, scale):
    """Scores [B, H, N, N] and values [B, H, N, dv] of the restatement."""
    _, q, k, qb, cb = mo.project(x, W_phi, gq, gk, H, m)
    return mo.scores(q, k, qb, cb, scale), mo.values(x, W_V, H)


@pytest.mark.parametrize("sgn", [1.0, -1.0])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("split", [1, 3])
def test_matches_reference_accumulators(sgn, causal, split):
    x, W_phi, gq, gk, W_V = _inputs(2, 6, 4, 2, 3, seed=1)
    out = mo.soft_morph_ref(x, W_phi, gq, gk, W_V, 0.35, 2, 3, scale=0.8, causal=causal, sgn=sgn)
    ref = torch.tensor(mo.soft_morph_brute_force(x, W_phi, gq, gk, W_V, 0.35, 2, 3, scale=0.8, causal=causal,
                                                 sgn=sgn, split=split), dtype=torch.float64)
    assert torch.allclose(out, ref, atol=1e-12, rtol=0)


@pytest.mark.parametrize("causal", [False, True])
def test_small_tau_is_the_hard_tropical_product(causal):
    """max_j x_j <= tau ln sum_j exp(x_j / tau) <= max_j x_j + tau ln n (and
    the mirror bound for the min-plus product)."""
    H, m, scale, tau = 2, 4, 0.9, 1e-3
    x, W_phi, gq, gk, W_V = _inputs(2, 9, 8, H, m, seed=2, x_mult=2.0)
    s, V = _sv(x, W_phi, gq, gk, W_V, H, m, scale)
    xs = s[..., :, :, None] + V[..., None, :, :]                     # [B, H, i, j, c]
    n = torch.ones(9, 9).sum(-1)
    if causal:
        xs_max = xs.masked_fill(mo.causal_mask(9, "cpu")[:, :, None], -math.inf).amax(-2)
        xs_min = xs.masked_fill(mo.causal_mask(9, "cpu")[:, :, None], math.inf).amin(-2)
        n = torch.arange(1, 10, dtype=torch.float64)
    else:
        xs_max, xs_min = xs.amax(-2), xs.amin(-2)
    slack = (tau * torch.log(n))[None, None, :, None]
    for sgn, hard in ((1.0, xs_max), (-1.0, xs_min)):
        out = mo.soft_morph_ref(x, W_phi, gq, gk, W_V, tau, H, m, scale=scale, causal=causal, sgn=sgn)
        o = out.view(2, 9, H, 4).permute(0, 2, 1, 3)
        dev = sgn * (o - hard)
        assert bool((dev >= -1e-12).all()) and bool((dev <= slack + 1e-12).all())


def test_large_tau_expansion_within_hoeffding_bound():
    """mean_j x_j <= tau ln(1/n sum_j exp(x_j / tau)) <= mean_j x_j + range^2 / (8 tau)."""
    H, m, scale, tau, N = 2, 3, 0.7, 50.0, 7
    x, W_phi, gq, gk, W_V = _inputs(1, N, 6, H, m, seed=3)
    s, V = _sv(x, W_phi, gq, gk, W_V, H, m, scale)
    xs = s[..., :, :, None] + V[..., None, :, :]
    out = mo.soft_morph_ref(x, W_phi, gq, gk, W_V, tau, H, m, scale=scale).view(1, N, H, 3).permute(0, 2, 1, 3)
    excess = out - tau * math.log(N) - xs.mean(-2)
    rng = xs.amax(-2) - xs.amin(-2)
    assert bool((excess >= -1e-12).all()) and bool((excess <= rng ** 2 / (8 * tau) + 1e-12).all())
    assert float(excess.max()) > 0  # the bound is not vacuous here


@pytest.mark.parametrize("causal", [False, True])
def test_erosion_is_dual_dilation(causal):
    """soft min-plus(s, V) = -soft max-plus(-s, -V); -s comes from -scale."""
    x, W_phi, gq, gk, W_V = _inputs(2, 8, 6, 2, 3, seed=4)
    ero = mo.soft_morph_ref(x, W_phi, gq, gk, W_V, 0.4, 2, 3, scale=0.6, causal=causal, sgn=-1.0)
    dil = mo.soft_morph_ref(x, W_phi, gq, gk, -W_V, 0.4, 2, 3, scale=-0.6, causal=causal, sgn=1.0)
    assert torch.allclose(ero, -dil, atol=1e-12, rtol=0)


def test_single_key_is_score_plus_value():
    x, W_phi, gq, gk, W_V = _inputs(3, 1, 4, 2, 3, seed=5)
    s, V = _sv(x, W_phi, gq, gk, W_V, 2, 3, 1.3)
    for sgn in (1.0, -1.0):
        out = mo.soft_morph_ref(x, W_phi, gq, gk, W_V, 0.25, 2, 3, scale=1.3, sgn=sgn)
        assert torch.allclose(out.view(3, 1, 2, 2).permute(0, 2, 1, 3), s + V, atol=1e-13, rtol=0)


def test_masked_diagonal_causal_empties_row_zero():
    x, W_phi, gq, gk, W_V = _inputs(1, 4, 4, 2, 3, seed=6)
    out, zb = mo.soft_morph_ref(x, W_phi, gq, gk, W_V, 0.5, 2, 3, causal=True, mask_diag=True, return_zb=True)
    assert bool((out[:, 0] == 0).all()) and bool((zb[:, 0] == -mo.FLT_MAX).all())
    assert bool(torch.isfinite(out).all())


def test_weights_are_a_partition_of_unity():
    """d out_ic / d V_jc = P_ijc with sum_j P_ijc = 1: for dO = 1 the value
    gradient sums to the number of queries in every column, and the score
    gradient of every row sums to dv."""
    H, m, N = 2, 3, 6
    x, W_phi, gq, gk, W_V = _inputs(1, N, 4, H, m, seed=7)
    s, V = _sv(x, W_phi, gq, gk, W_V, H, m, 0.8)
    s = s.detach().requires_grad_(True)
    V = V.detach().requires_grad_(True)
    for sgn in (1.0, -1.0):
        out = sgn * 0.3 * torch.logsumexp(sgn * (s[..., :, :, None] + V[..., None, :, :]) / 0.3, dim=-2)
        gs, gv = torch.autograd.grad(out.sum(), (s, V))
        assert torch.allclose(gv.sum(-2), torch.full_like(gv.sum(-2), float(N)), atol=1e-12)
        assert torch.allclose(gs.sum(-1), torch.full_like(gs.sum(-1), float(V.shape[-1])), atol=1e-12)


@pytest.mark.parametrize("sgn", [1.0, -1.0])
def test_tau_gradient_identity(sgn):
    """dL/dtau = (sum dO out - sum_ij ds_ij s_ij - sum_jc dV_jc V_jc) / tau,
    the form the kernels use (soft_morph.cuh:71-77 states the per-element
    term (out - sum_j P (s + v)) / tau)."""
    H, m, N = 2, 3, 7
    x, W_phi, gq, gk, W_V = _inputs(1, N, 4, H, m, seed=8)
    s, V = _sv(x, W_phi, gq, gk, W_V, H, m, 0.9)
    s = s.detach().requires_grad_(True)
    V = V.detach().requires_grad_(True)
    tau = torch.tensor(0.45, dtype=torch.float64, requires_grad=True)
    keep = ~mo.causal_mask(N, "cpu")
    y = (sgn * (s[..., :, :, None] + V[..., None, :, :]) / tau).masked_fill(~keep[:, :, None], -math.inf)
    out = sgn * tau * torch.logsumexp(y, dim=-2)
    dO = torch.randn(out.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(9))
    gs, gv, gt = torch.autograd.grad((out * dO).sum(), (s, V, tau))
    ident = ((dO * out).sum() - (gs * s.masked_fill(~keep, 0.0)).sum() - (gv * V).sum()) / tau
    assert abs((gt - ident).item()) < 1e-12


@pytest.mark.parametrize("sgn,causal", [(1.0, False), (-1.0, True)])
def test_gradcheck_fp64_including_tau(sgn, causal):
    x, W_phi, gq, gk, W_V = _inputs(2, 5, 4, 2, 3, seed=10)
    tau = torch.tensor(0.6, dtype=torch.float64)
    args = [t.clone().requires_grad_(True) for t in (x, W_phi, gq, gk, W_V, tau)]

    def f(x, W_phi, gq, gk, W_V, tau):
        return mo.soft_morph_ref(x, W_phi, gq, gk, W_V, tau, 2, 3, scale=0.7, causal=causal, sgn=sgn)

    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-7, rtol=1e-5)


def test_planted_log2_finalize_is_caught(monkeypatch):
    """A finalize in base 2 (tau * log2 l instead of tau * ln l) fails the
    small-tau bound."""
    real = torch.logsumexp
    monkeypatch.setattr(torch, "logsumexp", lambda t, dim: real(t, dim=dim) * mo.LOG2E)
    x, W_phi, gq, gk, W_V = _inputs(1, 9, 8, 2, 4, seed=2, x_mult=2.0)
    s, V = _sv(x, W_phi, gq, gk, W_V, 2, 4, 0.9)
    hard = (s[..., :, :, None] + V[..., None, :, :]).amax(-2)
    out = mo.soft_morph_ref(x, W_phi, gq, gk, W_V, 1e-3, 2, 4, scale=0.9)
    dev = out.view(1, 9, 2, 4).permute(0, 2, 1, 3) - hard
    assert not bool((dev.abs() <= 1e-3 * math.log(9) + 1e-12).all())

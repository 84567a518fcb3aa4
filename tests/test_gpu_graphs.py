"""HIP-graph capture of the library's forward + backward.

The C ABI launches kernels only: no memset, allocation or synchronisation
(fills are kernels), so a whole training step of the drop-in autograd path can
be captured once and replayed. Each replay is checked against the eager
result, with the program's own eager work and synchronisations between the
replays. The forward output must replay bit for bit. The dq accumulation uses
fp32 atomics, whose order varies between runs (an fp16 gradient element can
move by an ulp), so gradients are compared to a 2e-3 relative bar (two fp16
ulps of the largest element) instead of bitwise.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import morphottention_amd  # noqa: F401
    yield


def _inputs(B, N, H, m, dv, seed):
    from morphottention_amd import MorphoAttention
    torch.manual_seed(seed)
    mod = MorphoAttention(H * dv, H, m, dtype=torch.float16, device="cpu")
    params = [p.detach().cuda().requires_grad_(True) for p in (mod.W_phi, mod.gate_q, mod.gate_k, mod.W_V)]
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(B, N, H * dv, generator=g).half().cuda().requires_grad_(True)
    dout = torch.randn(B, N, H * dv, generator=g).half().cuda()
    return x, params, dout


def _rel(a, b):
    return ((a.float() - b.float()).abs().max() / b.float().abs().max().clamp_min(1e-30)).item()


def _capture_and_replay(step, n_replays=3, bitwise=False):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eager = [t.detach().clone() for t in step()]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    worst = 0.0
    for i in range(n_replays):
        graph.replay()
        torch.cuda.synchronize()
        # the forward has no atomics: its output replays bit for bit
        assert torch.equal(static[0], eager[0]), f"replay {i}: forward output differs from eager"
        rels = [_rel(s, e) for s, e in zip(static, eager)]
        print(f"[graph] replay {i}: max rel diff {max(rels):.2e}", flush=True)
        if bitwise:
            assert all(torch.equal(s, e) for s, e in zip(static, eager)), f"replay {i}: gradients differ from eager"
        worst = max(worst, max(rels))
        other = [t.detach().clone() for t in step()]  # eager work between the replays
        torch.cuda.synchronize()
        assert all(torch.isfinite(t).all() for t in other)
    return worst


@pytest.mark.parametrize("causal", [False, True])
def test_softmax_step_replays(causal):
    from morphottention_amd import MorphoAttentionFunction
    B, N, H, m, dv = 2, 256, 2, 16, 64
    x, params, dout = _inputs(B, N, H, m, dv, seed=20)
    leaves = [x, *params]

    def step():
        out = MorphoAttentionFunction.apply(x, *params, H, m, 0.8, causal)
        return [out, *torch.autograd.grad(out, leaves, dout)]

    assert _capture_and_replay(step) <= 2e-3


@pytest.mark.parametrize("causal", [False, True])
def test_deterministic_step_replays_bitwise(causal):
    """MORPHO_MODE_DETERMINISTIC under capture: its partial-sum buffers are
    written by kernels (no memset), and every replay's gradients equal the
    eager step's bit for bit."""
    from morphottention_amd import MorphoAttentionFunction
    from morphottention_amd.autograd import variant_bits
    B, N, H, m, dv = 2, 300, 2, 16, 64
    x, params, dout = _inputs(B, N, H, m, dv, seed=22)
    leaves = [x, *params]
    variant = variant_bits(deterministic=True)

    def step():
        out = MorphoAttentionFunction.apply(x, *params, H, m, 0.8, causal, variant)
        return [out, *torch.autograd.grad(out, leaves, dout)]

    assert _capture_and_replay(step, bitwise=True) == 0.0


def test_soft_step_replays():
    from morphottention_amd import SoftMorphAttentionFunction
    B, N, H, m, dv = 2, 256, 2, 16, 64
    x, params, dout = _inputs(B, N, H, m, dv, seed=21)
    tau = torch.tensor([0.5], dtype=torch.float32, device="cuda", requires_grad=True)
    leaves = [x, *params, tau]

    def step():
        out = SoftMorphAttentionFunction.apply(x, *params, tau, H, m, 0.8, True, 1)
        return [out, *torch.autograd.grad(out, leaves, dout)]

    assert _capture_and_replay(step) <= 2e-3

"""GPU checks of the layers around the hot path: the attn-bench caller wrapper
(attn-bench/src/layers/attention/morpho_attention.py:9-41), the autograd
formula registered on the op itself, and torch.compile tracing of both."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import morpho_oracle as mo

pytestmark = pytest.mark.gpu

GRAD_TOL = 1e-2


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import morphottention_amd  # noqa: F401  (fails loudly if the build is missing)
    torch.backends.cuda.matmul.allow_tf32 = False
    yield


def _rel(a, b):
    return (a.float() - b.float()).abs().max().item() / max(b.float().abs().max().item(), 1e-30)


def test_multihead_self_attention_matches_oracle_composite():
    """The wrapper's fp32 forward and backward against the fp32 oracle of the
    attention followed by the same output projection."""
    from morphottention_amd import morpho_attention
    from morphottention_amd.layers import MultiHeadSelfAttention
    B, N, D, H, m = 2, 130, 256, 4, 16
    torch.manual_seed(1100)
    layer = MultiHeadSelfAttention(D, H, cube_m=m, causal=True).cuda()
    x = torch.randn(B, N, D, device="cuda", requires_grad=True)
    print(f"[case] MultiHeadSelfAttention B={B} N={N} D={D} H={H} m={m} causal", flush=True)
    out, attn_weights = layer(x, x, x)
    assert attn_weights is None and out.dtype == torch.float32 and out.shape == (B, N, D)
    a = layer.attn
    with torch.no_grad():  # the wrapper is exactly cast -> attention -> cast -> projection (dropout 0)
        direct = layer.proj(morpho_attention(x.half(), a.W_phi, a.gate_q, a.gate_k, a.W_V, H, m,
                                             scale=layer.scale, causal=True).float())
    assert torch.equal(out.detach(), direct)
    dout = torch.randn_like(out)
    out.backward(dout)

    xr = x.detach().half().float().requires_grad_()
    pr = [p.detach().float().requires_grad_() for p in (a.W_phi, a.gate_q, a.gate_k, a.W_V)]
    wr = layer.proj.weight.detach().clone().requires_grad_()
    br = layer.proj.bias.detach().clone().requires_grad_()
    ref = F.linear(mo.morpho_attention_ref(xr, *pr, H, m, scale=layer.scale, causal=True), wr, br)
    ref.backward(dout)
    fwd = _rel(out.detach(), ref.detach())
    rels = [_rel(g, r) for g, r in zip((x.grad, a.W_phi.grad, a.gate_q.grad, a.gate_k.grad, a.W_V.grad,
                                        layer.proj.weight.grad, layer.proj.bias.grad),
                                       (xr.grad, *[p.grad for p in pr], wr.grad, br.grad))]
    print(f"[parity] MultiHeadSelfAttention: fwd max-rel {fwd:.2e} grads " + " ".join(f"{r:.2e}" for r in rels),
          flush=True)
    assert fwd <= 2e-3
    assert max(rels) <= GRAD_TOL


def _inputs(B, N, H, m, dv, seed):
    from morphottention_amd import MorphoAttention
    torch.manual_seed(seed)
    mod = MorphoAttention(H * dv, H, m, causal=True, dtype=torch.float16, device="cpu")
    params = [p.detach().cuda() for p in (mod.W_phi, mod.gate_q, mod.gate_k, mod.W_V)]
    torch.manual_seed(seed + 1)
    x = torch.randn(B, N, H * dv).half().cuda()
    dout = torch.randn(B, N, H * dv).half().cuda()
    return x, params, dout


def test_forward_op_autograd_matches_function():
    """out of torch.ops.morphottention.forward is differentiable; its
    gradients (reference-schema backward, recomputing the projection) agree
    with MorphoAttentionFunction's (workspace-carrying backward)."""
    from morphottention_amd import morpho_attention
    B, N, H, m, dv = 2, 200, 4, 16, 64
    x, params, dout = _inputs(B, N, H, m, dv, 1200)
    print(f"[case] op autograd B={B} N={N} H={H} m={m} dv={dv}", flush=True)
    la = [t.clone().requires_grad_() for t in (x, *params)]
    out_a, _ = torch.ops.morphottention.forward(*la, H, m, 1.0, True)
    out_a.backward(dout)
    lb = [t.clone().requires_grad_() for t in (x, *params)]
    out_b = morpho_attention(lb[0], *lb[1:], H, m, scale=1.0, causal=True)
    out_b.backward(dout)
    assert torch.equal(out_a, out_b)
    for a, b in zip(la, lb):
        assert (a.grad.float() - b.grad.float()).abs().max().item() <= 1e-3 * max(1.0, b.grad.float().abs().max().item())


def test_torch_compile_traces_module_and_op():
    """torch.compile (AOT autograd, eager kernels) traces MorphoAttention and
    the differentiable op with fullgraph=True; outputs equal the eager ones,
    gradients up to the summation order of the dq atomics."""
    from morphottention_amd import MorphoAttention
    B, N, H, m, dv = 2, 96, 2, 16, 64
    x, params, dout = _inputs(B, N, H, m, dv, 1300)
    print(f"[case] torch.compile aot_eager B={B} N={N} H={H} m={m} dv={dv}", flush=True)
    mod = MorphoAttention(H * dv, H, m, causal=True, dtype=torch.float16, device="cuda")
    with torch.no_grad():
        for p, v in zip((mod.W_phi, mod.gate_q, mod.gate_k, mod.W_V), params):
            p.copy_(v)
    xe = x.clone().requires_grad_()
    out_e = mod(xe)
    out_e.backward(dout)
    grads_e = [xe.grad] + [p.grad.clone() for p in mod.parameters()]
    mod.zero_grad()
    compiled = torch.compile(mod, backend="aot_eager", fullgraph=True)
    xc = x.clone().requires_grad_()
    out_c = compiled(xc)
    out_c.backward(dout)
    grads_c = [xc.grad] + [p.grad for p in mod.parameters()]
    assert torch.equal(out_c, out_e)
    for a, b in zip(grads_c, grads_e):  # dq is accumulated with atomics: equal up to summation order
        assert (a.float() - b.float()).abs().max().item() <= 1e-3 * max(1.0, b.float().abs().max().item())

    def op_out(x, W_phi, gate_q, gate_k, W_V):
        return torch.ops.morphottention.forward(x, W_phi, gate_q, gate_k, W_V, H, m, 1.0, True)[0]

    lo = [t.clone().requires_grad_() for t in (x, *params)]
    out_o = torch.compile(op_out, backend="aot_eager", fullgraph=True)(*lo)
    out_o.backward(dout)
    assert torch.equal(out_o, out_e)
    for a, b in zip(lo, grads_e):
        assert (a.grad.float() - b.float()).abs().max().item() <= 1e-3 * max(1.0, b.float().abs().max().item())

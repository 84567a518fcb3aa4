"""Host-side checks of the drop-in boundary (no GPU needed).

* the C-ABI library loads and exports every function ``include/*.h`` declares;
* argument validation returns the documented status codes and messages
  without touching a device;
* the torch op schemas equal the reference's
  (``packages/morphottention/csrc/cuda/binder.cpp:7-11``);
* fake (meta) kernels, module construction, init and errors mirror
  ``packages/morphottention/torch-ext/morphottention/autograd.py``.
"""

from __future__ import annotations

import ctypes
import glob
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    names = []
    for path in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(morpho_[a-z_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_entry_points():
    names = _header_functions()
    for required in ("morpho_forward", "morpho_backward", "morpho_forward_workspace_size",
                     "morpho_backward_workspace_size", "morpho_last_error", "morpho_status_string"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from morphottention_amd import capi
    L = capi.lib()
    for name in _header_functions():
        assert hasattr(L, name), name
        # and it is a real dynamic symbol of the library, not of a dependency
        assert ctypes.cast(getattr(L, name), ctypes.c_void_p).value


def test_status_strings_and_version():
    from morphottention_amd import capi
    L = capi.lib()
    assert L.morpho_version() >= 100
    assert L.morpho_status_string(0) == b"ok"
    assert L.morpho_status_string(3).startswith(b"workspace")


def test_workspace_sizes():
    from morphottention_amd import capi
    f = capi.forward_workspace_size(4, 4096, 1024, 16, 16)
    assert f > 4 * 4096 * 1024 * 2  # holds at least the per-head values
    b_with = capi.backward_workspace_size(4, 4096, 1024, 16, 16, True)
    b_without = capi.backward_workspace_size(4, 4096, 1024, 16, 16, False)
    assert b_without == b_with + f
    assert capi.forward_workspace_size(4, 4096, 1024, 16, 24) == 0      # unsupported cube_m
    assert capi.forward_workspace_size(4, 4096, 1000, 16, 16) == 0      # D % H != 0
    assert capi.forward_workspace_size(4, 4096, 256, 16, 16) == 0       # head_dim_v 16 unsupported
    # launch grids stay below 2^32 work-items: tokens <= 2^28, tokens x D <= 2^34,
    # tokens x H x cube_m <= 2^33 (each at its limit is accepted, one more token is not)
    assert capi.forward_workspace_size(1, 1 << 24, 1024, 16, 32) > 0    # T D = 2^34, T H m = 2^33
    assert capi.forward_workspace_size(1, (1 << 24) + 1, 1024, 16, 32) == 0
    assert capi.forward_workspace_size(1 << 14, 1 << 14, 64, 1, 16) > 0  # T = 2^28
    assert capi.forward_workspace_size((1 << 14) + 1, 1 << 14, 64, 1, 16) == 0
    assert capi.forward_workspace_size(1 << 40, 1 << 40, 64, 1, 16) == 0  # no int64 overflow in T


def _size_valid(B, N, D, H, m):
    """The documented size contract of the C ABI (include/morphottention.h)."""
    if min(B, N, D, H) <= 0 or D % H or m not in (16, 32, 64) or D // H not in (32, 64, 128):
        return False
    if B > 1 << 28 or N > 1 << 28:
        return False
    T = B * N
    return T <= 1 << 28 and D <= 65536 and H * m <= 65536 and T * D <= 1 << 34 and T * H * m <= 1 << 33


def test_workspace_sizes_follow_the_size_contract():
    """Property over 1000 random problems whose token counts sit at, one past,
    inside or far beyond the limit that binds for their head shape (plus
    zero, negative and unsupported sizes; about a quarter are valid, and an
    expected limit off by one token or by a factor of two fails the test):
    every workspace size function returns 0
    exactly when the documented contract is broken; otherwise the forward
    workspace holds at least the code rows, values, remainders, row
    statistics and weights it is carved into, the backward workspace without
    a forward one is the one with it plus the forward's, and the
    deterministic mode only adds to it."""
    from hypothesis import given, settings, strategies as st
    from morphottention_amd import capi

    @st.composite
    def problems(draw):
        # the head shape first, then a token count aimed at the limit that
        # binds for it (exactly at it, one past it, inside or far beyond), then
        # a split of the tokens into B x N (B a power of two, so an exact
        # limit stays exact); a few draws use degenerate sizes instead
        H = draw(st.sampled_from([1, 1, 1, 2, 3, 8, 16, 32, 512, 1 << 12, 1 << 20]))
        dv = draw(st.sampled_from([32, 64, 128] * 3 + [16, 96, 256]))
        m = draw(st.sampled_from([16, 32, 64] * 3 + [8, 24, 128]))
        if draw(st.integers(0, 9)) == 0:
            return draw(st.integers(-2, 2)), draw(st.integers(-2, 1 << 40)), H * dv, H, m
        tmax = min(1 << 28, (1 << 34) // (H * dv), (1 << 33) // (H * m))
        kind = draw(st.integers(0, 3))
        T = max(1, [tmax, tmax + 1, draw(st.integers(1, max(1, tmax))), draw(st.integers(tmax + 1, 8 * tmax + 8))][kind])
        B = 1 << draw(st.integers(0, max(0, min(40, T.bit_length() - 1))))
        return B, max(1, T // B), H * dv, H, m

    @settings(max_examples=1000, deadline=None, derandomize=True)
    @given(p=problems())
    def prop(p):
        B, N, D, H, m = p
        dv = D // H
        ok = _size_valid(B, N, D, H, m)
        f = capi.forward_workspace_size(B, N, D, H, m)
        bw = capi.backward_workspace_size(B, N, D, H, m, True)
        bwo = capi.backward_workspace_size(B, N, D, H, m, False)
        bd = capi.backward_workspace_size(B, N, D, H, m, True, mode=1 | 32)
        sf = capi.soft_forward_workspace_size(B, N, D, H, m)
        assert (f > 0) == ok and (bw > 0) == ok and (bwo > 0) == ok and (bd > 0) == ok and (sf > 0) == ok, \
            (B, N, D, H, m, f, bw, bwo, bd, sf)
        if ok:
            T = B * N
            NP = (N + 63) // 64 * 64
            carved = 2 * T * H * (2 * m + 8) * 2 + B * H * NP * dv * 3 + T * H * 16 + 2 * (H * m + D) * D * 2
            assert carved <= f < 2 ** 62
            assert bwo == bw + f and bd >= bw and sf >= f

    prop()


@pytest.mark.parametrize("D,H,m", [(1024, 16, 16), (2048, 32, 64)])
def test_backward_workspace_grows_only_with_per_token_buffers(D, H, m):
    """The weight gradient's per-piece partials (dW tiles x pieces x bt x bt
    fp32, at most one round of workgroups) do not grow with the token count:
    the backward workspace grows only by its per-token buffers (dZ|dV rows,
    dq, dk, dcb, the row sums, the dO affine rows and the per-block gate
    partials)."""
    from morphottention_amd import capi
    N = 4096
    HM, NC = H * m, H * m + D
    # bytes per token of the buffers that must scale with T (the gate partials
    # are one row of H m floats per 64 tokens)
    per_token = 2 * NC + H * 16 + 2 * 4 * HM + 4 * H + 8 * H + 4 * HM / 64
    w1 = capi.backward_workspace_size(64, N, D, H, m, True)
    w2 = capi.backward_workspace_size(256, N, D, H, m, True)
    assert w1 > 0 and w2 > 0
    grow = (w2 - w1) / (192 * N)
    assert grow <= per_token * 1.001 + 1, (grow, per_token)
    # and the partials stay small in absolute terms at a million tokens
    assert w2 - 256 * N * per_token < 512 << 20


def _call_forward(L, ptr, *, M=16, D=64, H=2, ws=1 << 20, mode=0):
    vp = ctypes.c_void_p(ptr)
    lse = ctypes.c_void_p(ptr)
    return L.morpho_forward(vp, vp, vp, vp, vp, vp, lse, 2, 8, D, H, M, 1.0, mode, vp, ws, None)


def test_forward_validation_never_reaches_the_device():
    from morphottention_amd import capi
    L = capi.lib()
    vp = ctypes.c_void_p(0)
    st = L.morpho_forward(vp, vp, vp, vp, vp, vp, vp, 2, 8, 64, 2, 16, 1.0, 0, vp, 0, None)
    assert st == 1 and L.morpho_last_error() == b"Null pointer"
    assert _call_forward(L, 4096, M=24) == 2
    assert b"cube_m" in L.morpho_last_error()
    assert _call_forward(L, 4096, D=63) == 1
    assert L.morpho_last_error() == b"D must be divisible by H"
    assert _call_forward(L, 4096, ws=16) == 3
    assert b"workspace" in L.morpho_last_error()
    assert _call_forward(L, 4100) == 1  # misaligned
    for bad in (16, 12, 13, 0x100):  # an unknown bit; both projections
        assert _call_forward(L, 4096, mode=bad) == 1
        assert b"invalid mode bits" in L.morpho_last_error()
    st = L.morpho_backward(*([vp] * 13), 2, 8, 64, 2, 16, 1.0, 0, None, vp, 0, None)
    assert st == 1 and L.morpho_last_error() == b"Null input pointer"


# (N, D, H, m): keys per backward key block KW and query step QT of the
# kernel configuration, which fix the size of the deterministic partials
DET_LAYOUTS = [((4, 4096, 1024, 16, 16), 128, 64), ((1, 16384, 1024, 16, 32), 256, 32),
               ((16, 2048, 2048, 32, 64), 256, 32), ((2, 1000, 1024, 8, 32), 128, 32),
               ((3, 777, 512, 8, 16), 128, 64), ((1, 1, 64, 2, 64), 256, 32)]


@pytest.mark.parametrize("shape,kw,qt", DET_LAYOUTS, ids=lambda v: str(v))
def test_deterministic_workspace_adds_the_partials(shape, kw, qt):
    """MORPHO_MODE_DETERMINISTIC adds [nkb, B*H, NQ, M] + [nkb, B*H, NQ] fp32
    partials (nkb = ceil(N / KW) key blocks, NQ = N rounded up to the query
    step), each 256-byte aligned; no other mode bit changes the size."""
    from morphottention_amd import capi
    B, N, D, H, m = shape
    al = lambda n: (n + 255) // 256 * 256  # noqa: E731
    nkb, nq = -(-N // kw), -(-N // qt) * qt
    rows = nkb * B * H * nq
    for have_fwd in (True, False):
        base = capi.backward_workspace_size(B, N, D, H, m, have_fwd)
        for mode in (0, 1, 2, 3, 4, 9):
            assert capi.backward_workspace_size(B, N, D, H, m, have_fwd, mode) == base
        for mode in (32, 33, 38):
            assert capi.backward_workspace_size(B, N, D, H, m, have_fwd, mode) == base + al(rows * m * 4) + al(rows * 4)
        assert capi.backward_workspace_size(B, N, D, H, m, have_fwd, 64) == 0      # unknown bit
        assert capi.backward_workspace_size(B, N, D, H, m, have_fwd, 32 | 12) == 0  # two projections


def test_deterministic_mode_bit_is_plumbed():
    from morphottention_amd import MorphoAttention
    from morphottention_amd.autograd import variant_bits
    assert variant_bits(deterministic=True) == 32
    assert variant_bits("identity", True, True) == 8 | 2 | 32
    mod = MorphoAttention(64, 2, 16, device="cpu", deterministic=True)
    assert mod.variant == 32 and mod.deterministic
    # the size query keeps the thread's last error, like the other size queries
    from morphottention_amd import capi
    L = capi.lib()
    vp = ctypes.c_void_p(0)
    L.morpho_forward(vp, vp, vp, vp, vp, vp, vp, 2, 8, 64, 2, 16, 1.0, 0, vp, 0, None)
    assert capi.backward_workspace_size(2, 8, 64, 2, 16, True, 32) > 0
    assert L.morpho_last_error() == b"Null pointer"


REF_SCHEMAS = {
    "forward": "morphottention::forward(Tensor X, Tensor W_phi, Tensor gate_q, Tensor gate_k, Tensor W_V, "
               "int H, int cube_m, float scale, bool causal) -> Tensor[]",
    "backward": "morphottention::backward(Tensor grad_out, Tensor X, Tensor W_phi, Tensor gate_q, Tensor gate_k, "
                "Tensor W_V, Tensor out, Tensor lse, int H, int cube_m, float scale, bool causal) -> Tensor[]",
}


@pytest.mark.parametrize("name", sorted(REF_SCHEMAS))
def test_op_schemas_match_reference(name):
    import morphottention_amd  # noqa: F401
    assert str(getattr(torch.ops.morphottention, name).default._schema) == REF_SCHEMAS[name]


def test_fake_kernels():
    import morphottention_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    ops = torch.ops.morphottention
    with FakeTensorMode():
        X = torch.empty(2, 8, 64, dtype=torch.float16, device="cuda")
        W = torch.empty(64, 32, dtype=torch.float16, device="cuda")
        g = torch.empty(2, 16, dtype=torch.float16, device="cuda")
        V = torch.empty(64, 64, dtype=torch.float16, device="cuda")
        out, lse = ops.forward(X, W, g, g, V, 2, 16, 1.0, True)
        assert out.shape == X.shape and lse.shape == (4, 8) and lse.dtype == torch.float32
        out2, lse2, ws = ops.forward_train(X, W, g, g, V, 2, 16, 1.0, True)
        assert ws.dtype == torch.uint8 and ws.numel() > 0
        grads = ops.backward(out, X, W, g, g, V, out, lse, 2, 16, 1.0, True)
        assert [t.shape for t in grads] == [X.shape, W.shape, g.shape, g.shape, V.shape]
        grads = ops.backward_train(out, X, W, g, g, V, out, lse, ws, 2, 16, 1.0, True)
        assert [t.shape for t in grads] == [X.shape, W.shape, g.shape, g.shape, V.shape]


def test_reference_import_path():
    """The reference's import line works unchanged
    (torch-ext/morphottention/__init__.py:1-3; attn-bench's morpho_attention.py:7),
    with the same public names and submodules, and resolves to this build."""
    import morphottention
    from morphottention import MorphoAttention, MorphoAttentionFunction, morpho_attention
    from morphottention._ops import add_op_namespace_prefix, ops
    import morphottention_amd
    assert morphottention.__all__ == ["MorphoAttention", "MorphoAttentionFunction", "morpho_attention"]
    assert MorphoAttention is morphottention_amd.MorphoAttention
    assert MorphoAttentionFunction is morphottention_amd.MorphoAttentionFunction
    assert morpho_attention is morphottention_amd.morpho_attention
    assert morphottention.autograd.MorphoAttention is MorphoAttention
    assert ops is torch.ops.morphottention and add_op_namespace_prefix("forward") == "morphottention::forward"
    # the reference autograd's fallback loader name (autograd.py:10-13, _cmake_ops.py:15-30)
    from morphottention._cmake_ops import add_op_namespace_prefix as prefix2, ops as ops2
    assert ops2 is ops and prefix2 is add_op_namespace_prefix
    mod = MorphoAttention(64, 2, 16, dtype=torch.float16, device="cpu")
    with pytest.raises(ValueError, match="CUDA tensor"):
        mod(torch.randn(1, 4, 64, dtype=torch.float16))


def test_module_construction_and_init_protocol():
    from morphottention_amd import MorphoAttention
    torch.manual_seed(0)
    mod = MorphoAttention(256, 8, 16, scale=0.5, causal=True, dtype=torch.float32, device="cpu")
    assert set(dict(mod.named_parameters())) == {"W_phi", "gate_q", "gate_k", "W_V"}
    assert mod.W_phi.shape == (256, 128) and mod.W_V.shape == (256, 256)
    assert mod.gate_q.shape == (8, 16) and torch.equal(mod.gate_k, torch.ones(8, 16))
    torch.manual_seed(0)
    a = torch.empty(256, 128).normal_(0.0, 256 ** -0.5)
    b = torch.empty(256, 256).normal_(0.0, 256 ** -0.5)
    assert torch.equal(mod.W_phi.detach(), a) and torch.equal(mod.W_V.detach(), b)
    with pytest.raises(ValueError, match="divisible"):
        MorphoAttention(250, 8, 16)


def test_cpu_input_raises_value_error():
    from morphottention_amd import MorphoAttention, morpho_attention
    mod = MorphoAttention(64, 2, 16, dtype=torch.float16, device="cpu")
    x = torch.randn(1, 4, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="CUDA tensor"):
        mod(x)
    with pytest.raises(ValueError, match="CUDA tensor"):
        morpho_attention(x, mod.W_phi, mod.gate_q, mod.gate_k, mod.W_V, 2, 16)


def test_raw_op_on_cpu_tensors_is_not_silently_computed():
    import morphottention_amd  # noqa: F401
    X = torch.randn(1, 4, 64, dtype=torch.float16)
    W = torch.randn(64, 32, dtype=torch.float16)
    g = torch.ones(2, 16, dtype=torch.float16)
    V = torch.randn(64, 64, dtype=torch.float16)
    with pytest.raises((NotImplementedError, RuntimeError)):
        torch.ops.morphottention.forward(X, W, g, g, V, 2, 16, 1.0, False)


def test_forward_op_is_differentiable_under_fake_tensors():
    """torch.ops.morphottention.forward carries its own autograd formula (the
    reference-schema backward op); under fake tensors the graph forms and
    every differentiable input receives a gradient of its own shape."""
    import morphottention_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        B, N, D, H, m = 2, 64, 128, 2, 16
        x = torch.empty(B, N, D, dtype=torch.float16).requires_grad_()
        W = torch.empty(D, H * m, dtype=torch.float16).requires_grad_()
        gq = torch.empty(H, m, dtype=torch.float16).requires_grad_()
        gk = torch.empty(H, m, dtype=torch.float16).requires_grad_()
        V = torch.empty(D, D, dtype=torch.float16).requires_grad_()
        out, lse = torch.ops.morphottention.forward(x, W, gq, gk, V, H, m, 1.0, True)
        assert out.grad_fn is not None
        out.sum().backward()
        for t in (x, W, gq, gk, V):
            assert t.grad is not None and t.grad.shape == t.shape


def test_multihead_self_attention_wrapper_contract():
    """attn-bench's MultiHeadSelfAttention (attn-bench/src/layers/attention/
    morpho_attention.py:9-41): constructor defaults, attributes, parameters."""
    from morphottention_amd.layers import MultiHeadSelfAttention
    layer = MultiHeadSelfAttention(256, 4)
    assert layer.name == "morpho_attention"
    assert (layer.num_heads, layer.head_dim, layer.cube_m, layer.causal) == (4, 64, 64, False)
    assert layer.scale == 64 ** -0.5
    assert MultiHeadSelfAttention.HEAD_DIM == 64 and MultiHeadSelfAttention.CUBE_M == 64
    assert set(dict(layer.named_parameters())) == {"attn.W_phi", "attn.gate_q", "attn.gate_k", "attn.W_V",
                                                   "proj.weight", "proj.bias"}
    assert layer.attn.W_phi.dtype == torch.float16 and layer.proj.weight.dtype == torch.float32
    layer2 = MultiHeadSelfAttention(128, 2, 0.1, cube_m=16, scale=0.5, causal=True, unused_option=3)
    assert (layer2.cube_m, layer2.scale, layer2.causal) == (16, 0.5, True)
    assert layer2.attn.W_phi.shape == (128, 32) and layer2.dropout.p == 0.1
    x = torch.randn(1, 8, 128)
    with pytest.raises(ValueError, match="CUDA tensor"):
        layer2(x, x, x)


def test_soft_entry_points_validate_without_the_device():
    from morphottention_amd import capi
    L = capi.lib()
    vp = ctypes.c_void_p(4096)
    ws = 1 << 20
    # sgn must be +-1; tau must be given
    st = L.morpho_soft_forward(vp, vp, vp, vp, vp, vp, vp, vp, 2, 8, 64, 2, 16, 1.0, 0, 2, vp, ws, None)
    assert st == 1 and b"sgn" in L.morpho_last_error()
    st = L.morpho_soft_forward(vp, vp, vp, vp, vp, None, vp, vp, 2, 8, 64, 2, 16, 1.0, 0, 1, vp, ws, None)
    assert st == 1 and b"tau" in L.morpho_last_error()
    st = L.morpho_soft_forward(vp, vp, vp, vp, vp, vp, vp, vp, 2, 8, 64, 2, 16, 1.0, 64, 1, vp, ws, None)
    assert st == 1 and b"invalid mode bits" in L.morpho_last_error()  # 16 (SOFT_EXACT) is valid here, 64 is not
    st = L.morpho_soft_forward(vp, vp, vp, vp, vp, vp, vp, vp, 2, 8, 64, 2, 16, 1.0, 32, 1, vp, ws, None)
    assert st == 2 and b"softmax backward only" in L.morpho_last_error()  # DETERMINISTIC
    st = L.morpho_soft_backward(*([vp] * 14), 2, 8, 64, 2, 16, 1.0, 33, 1, None, vp, ws, None)
    assert st == 2 and b"softmax backward only" in L.morpho_last_error()
    st = L.morpho_soft_forward(vp, vp, vp, vp, vp, vp, vp, vp, 2, 8, 64, 2, 16, 1.0, 16, 1, vp, 64, None)
    assert st == 3 and b"soft forward workspace" in L.morpho_last_error()
    st = L.morpho_soft_backward(*([vp] * 14), 2, 8, 64, 2, 16, 1.0, 0, -3, None, vp, ws, None)
    assert st == 1 and b"sgn" in L.morpho_last_error()
    need_fwd = capi.soft_backward_workspace_size(2, 8, 64, 2, 16, True)
    assert need_fwd > capi.backward_workspace_size(2, 8, 64, 2, 16, True)
    assert capi.soft_backward_workspace_size(2, 8, 64, 2, 16, False) == need_fwd + capi.forward_workspace_size(
        2, 8, 64, 2, 16)
    assert capi.soft_backward_workspace_size(2, 8, 64, 2, 24, True) == 0


def test_soft_fake_kernels_and_module():
    import morphottention_amd  # noqa: F401
    from morphottention_amd import SoftMorphAttention
    from torch._subclasses.fake_tensor import FakeTensorMode
    ops = torch.ops.morphottention
    with FakeTensorMode():
        X = torch.empty(2, 8, 64, dtype=torch.float16, device="cuda")
        W = torch.empty(64, 32, dtype=torch.float16, device="cuda")
        g = torch.empty(2, 16, dtype=torch.float16, device="cuda")
        V = torch.empty(64, 64, dtype=torch.float16, device="cuda")
        t = torch.empty(1, dtype=torch.float32, device="cuda")
        out, zb, ws = ops.soft_forward(X, W, g, g, V, t, 2, 16, 1.0, True, 1)
        assert out.shape == X.shape and zb.shape == (4, 8, 32) and zb.dtype == torch.float32
        grads = ops.soft_backward(out, X, W, g, g, V, t, zb, ws, 2, 16, 1.0, True, -1)
        assert [x.shape for x in grads] == [X.shape, W.shape, g.shape, g.shape, V.shape, t.shape]
    mod = SoftMorphAttention(64, 2, 16, tau=0.3, erosion=True, dtype=torch.float32, device="cpu")
    assert set(dict(mod.named_parameters())) == {"W_phi", "gate_q", "gate_k", "W_V", "tau"}
    assert mod.sgn == -1 and mod.tau.dtype == torch.float32 and float(mod.tau) == pytest.approx(0.3)
    fixed = SoftMorphAttention(64, 2, 16, learn_tau=False, device="cpu")
    assert "tau" not in dict(fixed.named_parameters()) and "tau" in dict(fixed.named_buffers())
    with pytest.raises(ValueError, match="tau"):
        SoftMorphAttention(64, 2, 16, tau=0.0)
    with pytest.raises(ValueError, match="CUDA tensor"):
        mod(torch.randn(1, 4, 64))


def test_bench_work_counts_match_the_survey_table():
    """bench.py's algorithmic counts, which set roofline.achieved and the step
    fraction, against the independently computed table of the measurement
    plan (pairs P, F_fwd and F_bwd in GFLOP, MFMA-ideal times at 2.5 PFLOP/s,
    the C3 exp bound and compulsory bytes), to the table's printed digits."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    table = {  # cfg: (P, F_fwd, F_bwd, ideal fwd ms, ideal fwd+bwd ms)
        "C2": (6.71e7, 16.11, 34.36, 0.0064, 0.0202),
        "C3": (5.37e8, 128.87, 274.92, 0.0515, 0.1615),
        "C4": (2.15e9, 463.88, 1065.21, 0.1856, 0.6116),
        "C5": (2.15e9, 1099.51, 2473.90, 0.4398, 1.4294),
    }
    for cfg, (P, ff, fb, tf, tfb) in table.items():
        B, N, D, H, m, _scale, causal = bench.CONFIGS[cfg][:7]
        p = bench.pairs(B, N, H, causal)
        f_fwd, f_bwd = bench.step_flops(B, N, D, H, m, causal)
        assert abs(p - P) <= 0.005 * P, cfg
        assert round(f_fwd / 1e9, 2) == pytest.approx(ff, abs=0.011), cfg
        assert round(f_bwd / 1e9, 2) == pytest.approx(fb, abs=0.011), cfg
        assert round(f_fwd / 2.5e15 * 1e3, 4) == pytest.approx(tf, abs=1e-4), cfg
        assert round((f_fwd + f_bwd) / 2.5e15 * 1e3, 4) == pytest.approx(tfb, abs=1e-4), cfg
        # the per-kernel counts add up to the step's
        k = lambda n: bench.kernel_flops(n, B, N, D, H, m, causal)  # noqa: E731
        assert k("proj_fwd") + k("attn_fwd") == pytest.approx(f_fwd, rel=1e-12)
        assert k("attn_bwd") + k("bwd_gemm") == pytest.approx(f_bwd, rel=1e-12)
    B, N, D, H, m, _scale, causal = bench.CONFIGS["C3"][:7]
    assert bench.kernel_flops("attn_bwd", B, N, D, H, m, causal) / 1e9 == pytest.approx(189.0, abs=0.5)
    bound, t = bench.roofline_terms(*bench.step_flops(B, N, D, H, m, causal)[:1], bench.pairs(B, N, H, causal),
                                    bench.compulsory_bytes(B, N, D, H, m)[0])
    assert bound == "exp" and t["exp"] == pytest.approx(0.0548, abs=1e-4) and t["mfma"] == pytest.approx(0.0515, abs=1e-4)
    fwd_b, bwd_b = bench.compulsory_bytes(B, N, D, H, m)
    assert fwd_b / 1e6 == pytest.approx(70.8, abs=0.1) and bwd_b / 1e6 == pytest.approx(140.5, abs=0.1)

"""The allocation-free forward (morpho_forward_noalloc) through the C ABI:
two calls in a row, the second with a smaller problem, each bit-identical to
morpho_forward with a caller-owned workspace (the same kernels on the same
inputs), and an over-size problem refused before anything runs; and, in a
process of its own, a first call made under HIP graph capture
(tests/noalloc_capture_child.py)."""

from __future__ import annotations

import ctypes
import os
import subprocess
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(B, N, D, H, m, seed):
    from morphottention_amd import MorphoAttention
    torch.manual_seed(seed)
    mod = MorphoAttention(D, H, m, dtype=torch.float16, device="cpu")
    params = [mod.W_phi.detach(), mod.gate_q.detach(), mod.gate_k.detach(), mod.W_V.detach()]
    x = torch.randn(B, N, D).half()
    return x.cuda(), [p.cuda().contiguous() for p in params]


def test_forward_noalloc_matches_forward():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    from morphottention_amd import capi
    L = capi.lib()
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # the first call fills 28 of the 32 MiB scratch array, the second is
    # smaller and ragged (causal, masked diagonal: a keyless row), so stale
    # bytes of the first call lie beyond what the second writes; the reference
    # workspace is filled with 0xFF bytes, so a kernel that read a byte its
    # call never wrote would differ between the two
    for (B, N, D, H, m, mode, seed) in [(1, 4096, 1024, 16, 16, 1, 1), (1, 300, 256, 4, 32, 3, 2)]:
        x, params = _inputs(B, N, D, H, m, seed)
        need = capi.forward_workspace_size(B, N, D, H, m)
        print(f"[case] noalloc B={B} N={N} D={D} H={H} m={m} mode={mode} workspace {need} bytes", flush=True)
        assert 0 < need <= 32 << 20
        out = torch.empty_like(x)
        lse = torch.empty(B * H, N, dtype=torch.float32, device="cuda")
        st = L.morpho_forward_noalloc(*(vp(t) for t in (x, *params)), vp(out), vp(lse), B, N, D, H, m, 0.9, mode,
                                      stream)
        assert st == 0, L.morpho_last_error()
        ws = torch.full((need,), 0xFF, dtype=torch.uint8, device="cuda")
        ref_out = torch.empty_like(x)
        ref_lse = torch.empty_like(lse)
        st = L.morpho_forward(*(vp(t) for t in (x, *params)), vp(ref_out), vp(ref_lse), B, N, D, H, m, 0.9, mode,
                              vp(ws), need, stream)
        assert st == 0, L.morpho_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)
    # a problem beyond the scratch array is refused with a clear message
    B, N, D, H, m = 4, 4096, 1024, 16, 16
    st = L.morpho_forward_noalloc(*([ctypes.c_void_p(16)] * 7), B, N, D, H, m, 1.0, 1, stream)
    assert st == 3 and b"morpho_forward_noalloc" in L.morpho_last_error()


def test_first_noalloc_call_under_graph_capture():
    """The per-device scratch lookup happens on the first call; that call may
    be under stream capture. Run in a fresh process so that it is the first."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_capture_child.py")
    print("[case] noalloc first call under graph capture (child process)", flush=True)
    r = subprocess.run([sys.executable, child], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=180)
    print(r.stdout[-3000:], flush=True)
    assert r.returncode == 0 and "noalloc capture ok" in r.stdout

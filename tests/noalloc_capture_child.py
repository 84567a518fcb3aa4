"""Child process of tests/test_zz_no_alloc.py (run on its own, so that its
morpho_forward_noalloc call is the first of the process on the GPU).

1. The kernels are loaded by one morpho_forward with a caller workspace.
2. The first morpho_forward_noalloc call of the process (the per-device
   address lookup of the library's scratch array included) is made inside
   torch.cuda.graph capture.
3. The graph is replayed three times, with eager work between the replays;
   every replay must equal the eager morpho_forward bit for bit.
4. Around a further eager call neither torch's reserved memory nor the
   device's free memory (hipMemGetInfo) changes: nothing is allocated.
Prints "noalloc capture ok" and exits 0 on success.
"""

from __future__ import annotations

import ctypes
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import torch  # noqa: E402


def main() -> int:
    from morphottention_amd import MorphoAttention, capi
    L = capi.lib()
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    B, N, D, H, m, mode = 2, 777, 512, 8, 16, 1
    torch.manual_seed(5)
    mod = MorphoAttention(D, H, m, dtype=torch.float16, device="cpu")
    params = [p.detach().cuda().contiguous() for p in (mod.W_phi, mod.gate_q, mod.gate_k, mod.W_V)]
    x = torch.randn(B, N, D).half().cuda()
    need = capi.forward_workspace_size(B, N, D, H, m)
    ws = torch.full((need,), 0xFF, dtype=torch.uint8, device="cuda")
    ref_out, out = torch.empty_like(x), torch.empty_like(x)
    ref_lse = torch.empty(B * H, N, dtype=torch.float32, device="cuda")
    lse = torch.empty_like(ref_lse)
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731

    st = L.morpho_forward(*(vp(t) for t in (x, *params)), vp(ref_out), vp(ref_lse), B, N, D, H, m, 0.7, mode,
                          vp(ws), need, cur())
    assert st == 0, L.morpho_last_error()
    torch.cuda.synchronize()
    print("[child] eager morpho_forward done; capturing the first noalloc call", flush=True)

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = L.morpho_forward_noalloc(*(vp(t) for t in (x, *params)), vp(out), vp(lse), B, N, D, H, m, 0.7, mode,
                                      cur())
    assert st == 0, L.morpho_last_error()
    torch.cuda.synchronize()
    for i in range(3):
        out.zero_()
        lse.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse), f"replay {i} differs from eager"
        # eager work between replays: the workspace path again on poisoned memory
        ws.fill_(0xFF)
        st = L.morpho_forward(*(vp(t) for t in (x, *params)), vp(ref_out), vp(ref_lse), B, N, D, H, m, 0.7, mode,
                              vp(ws), need, cur())
        assert st == 0, L.morpho_last_error()
        torch.cuda.synchronize()
        print(f"[child] replay {i} bit-identical", flush=True)

    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    res0 = torch.cuda.memory_reserved()
    st = L.morpho_forward_noalloc(*(vp(t) for t in (x, *params)), vp(out), vp(lse), B, N, D, H, m, 0.7, mode, cur())
    assert st == 0, L.morpho_last_error()
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    res1 = torch.cuda.memory_reserved()
    assert free1 == free0 and res1 == res0, f"memory changed: free {free0} -> {free1}, reserved {res0} -> {res1}"
    assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)
    print("noalloc capture ok", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Generate the committed golden fixtures ``tests/golden/*.npz``.

The reference ships no golden vectors (its ``tests/`` package is empty), so
these fixtures come from the oracle (``oracle/morpho_oracle.py``) evaluated in
fp64 on fp16-representable inputs. The oracle is pinned independently by
``tests/test_oracle.py`` (gradcheck, SDPA equivalence, brute force, closed
forms); the fixtures freeze its values so that a later edit of the oracle, or
the HIP path on the GPU, is checked against fixed numbers.

Run from the repo root:  ``python tests/golden/make_golden.py``
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.morpho_oracle import init_params, morpho_attention_ref_grads  # noqa: E402

# name: (B, N, D, H, m, scale, causal, seed, x_mult, gates, dout_ones)
# gates: None for the default init (ones), else (mean, std) of random gates.
CASES = {
    # BASELINE configs[0] protocol (dim 256, 8 heads, m 16, B 2, N 128, seed 0,
    # backward of out.sum()).
    "c1_cpu_config": (2, 128, 256, 8, 16, 1.0, False, 0, 1.0, None, True),
    # Ragged length, causal, m = 32, non-unit gates.
    "causal_ragged_m32": (1, 77, 128, 2, 32, 0.5, True, 11, 1.0, (1.0, 0.5), False),
    # Wide cube, large-magnitude inputs, non-causal.
    "wide_m64_x4": (2, 40, 128, 2, 64, 2.0, False, 12, 4.0, None, False),
    # head_dim_v = 128, causal, gates with mixed signs.
    "dv128_causal": (1, 64, 256, 2, 16, 1.0, True, 13, 1.0, (0.0, 1.0), False),
}


def make_case(B, N, D, H, m, scale, causal, seed, x_mult, gates, dout_ones):
    torch.manual_seed(seed)
    W_phi, gate_q, gate_k, W_V = init_params(D, H, m)
    if gates is not None:
        gate_q = gates[0] + gates[1] * torch.randn(H, m)
        gate_k = gates[0] + gates[1] * torch.randn(H, m)
    torch.manual_seed(seed)
    x = x_mult * torch.randn(B, N, D)
    torch.manual_seed(seed + 1000)
    dout = torch.ones(B, N, D) if dout_ones else torch.randn(B, N, D)
    h = lambda t: t.to(torch.float16)  # noqa: E731
    x, W_phi, gate_q, gate_k, W_V, dout = map(h, (x, W_phi, gate_q, gate_k, W_V, dout))
    out, lse, grads = morpho_attention_ref_grads(
        x, W_phi, gate_q, gate_k, W_V, H, m, scale=scale, causal=causal, dout=dout, dtype=torch.float64)
    f16 = lambda t: t.numpy().astype(np.float16)  # noqa: E731
    f32 = lambda t: t.numpy().astype(np.float32)  # noqa: E731
    return dict(
        B=B, N=N, D=D, H=H, cube_m=m, scale=scale, causal=int(causal),
        x=f16(x), W_phi=f16(W_phi), gate_q=f16(gate_q), gate_k=f16(gate_k), W_V=f16(W_V), dout=f16(dout),
        out=f32(out), lse=f32(lse), dX=f32(grads[0]), dW_phi=f32(grads[1]), d_gate_q=f32(grads[2]),
        d_gate_k=f32(grads[3]), dW_V=f32(grads[4]),
    )


def main():
    for name, spec in CASES.items():
        data = make_case(*spec)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **data)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()

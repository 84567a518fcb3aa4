"""Error budget of the soft-hypercube (phi-path) gradients from the HIP
backward's fp16 storage points, evaluated in fp64 on the CPU.

With saturated codes and one-hot attention (inputs x4, cube_m 64, scale 2)
these gradients are sums of tiny terms that mostly cancel (~1e-7 of the
value-path gradients), and fp16 storage of two intermediates decides their
accuracy:
  * dS = P (dP - delta), rounded to fp16 before the code-gradient products
    (dq = dS phi_hi, dk = dS^T phi_hi, dcb = column sums);
  * dZ = dphi phi (1 - phi), rounded to fp16 into the [dZ | dV] operand of the
    weight-gradient GEMM.
Off-diagonal weights of one-hot rows make both fall into fp16's subnormal
range, where its relative precision is lost. ``phi_path_budget`` follows the
backward's arithmetic (tests' restatement of the math in the oracle, not the
oracle itself): fp64 everywhere except at those storage points, delta from the
fp16 output with the diagonal row-sum correction, and the fp16 rounding of the
returned gradients. The GPU parity test bounds the HIP error on such inputs by
this budget.
"""

from __future__ import annotations

import numpy as np
import torch


def _h16(t: torch.Tensor) -> torch.Tensor:
    return t.half().double()


def phi_gradients(x, W_phi, gate_q, gate_k, W_V, dout, H, m, scale, *, fp16_points=True):
    """dW_phi, d_gate_q, d_gate_k of one non-causal softmax attention call
    (sigmoid projection, diagonal in the softmax), in fp64. With
    ``fp16_points`` the backward's fp16 storage points are applied."""
    f = torch.float64
    X, Wp, WV = x.to(f), W_phi.to(f), W_V.to(f)
    gq, gk, dO = gate_q.to(f), gate_k.to(f), dout.to(f)
    B, N, D = X.shape
    dv = D // H
    dWp = torch.zeros_like(Wp)
    dG = torch.zeros(H, m, dtype=f)
    r16 = _h16 if fp16_points else (lambda t: t)
    for b in range(B):
        for h in range(H):
            phi = torch.sigmoid(X[b] @ Wp[:, h * m:(h + 1) * m])
            G = gq[h] * gk[h]
            s = -scale * (G * (phi[:, None, :] + phi[None, :, :] - 2 * phi[:, None, :] * phi[None, :, :])).sum(-1)
            P = torch.softmax(s, -1)
            V = X[b] @ WV[:, h * dv:(h + 1) * dv]
            out = r16(P @ V)  # the forward's fp16 output feeds delta
            do = dO[b][:, h * dv:(h + 1) * dv]
            dS = r16(P * (do @ V.T - (do * out).sum(-1)[:, None]))
            ph = r16(phi)  # the MFMA operand (phi_hi)
            dq, dk, dcb, r = dS @ ph, dS.T @ ph, dS.sum(0), dS.sum(1)
            # diagonal row-sum correction: dS_tt -> dS_tt - r_t P_tt
            c = r * P.diagonal()
            dq, dk, dcb, r = dq - c[:, None] * ph, dk - c[:, None] * ph, dcb - c, r - c
            dphi = scale * G * (2 * (dq + dk) - dcb[:, None] - r[:, None])
            dZ = r16(dphi * phi * (1 - phi))
            dWp[:, h * m:(h + 1) * m] += X[b].T @ dZ
            dG[h] += scale * (phi * (2 * dk - dcb[:, None])).sum(0)
    return [r16(dWp), r16(dG * gk), r16(dG * gq)]


def phi_path_budget(fixture: str) -> dict:
    """Relative max-norm error of each phi-path gradient against the
    fixture's fp64 values when only the fp16 storage points differ."""
    d = np.load(fixture)
    t = {k: torch.from_numpy(d[k]) for k in ("x", "W_phi", "gate_q", "gate_k", "W_V", "dout")}
    assert not bool(d["causal"])
    g = phi_gradients(t["x"], t["W_phi"], t["gate_q"], t["gate_k"], t["W_V"], t["dout"], int(d["H"]),
                      int(d["cube_m"]), float(d["scale"]))
    out = {}
    for n, v in zip(("dW_phi", "d_gate_q", "d_gate_k"), g):
        ref = torch.from_numpy(d[n]).double()
        out[n] = ((v - ref).abs().max() / ref.abs().max()).item()
    return out

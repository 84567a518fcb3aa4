"""CPU/eager restatement of the Morphottention attention math -- TEST INFRASTRUCTURE ONLY.

This module is the parity oracle for the HIP hot path. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only as the checker (or as the timed CPU baseline). The product path in
``morphottention_amd`` never routes through it.

It restates, in plain eager PyTorch (fp32 or fp64), the algorithm of the
reference CUDA extension (paths relative to the reference repo root):

* projection   ``packages/morphottention/csrc/cuda/sm120/project.cuh:26-45``
  (``Z = X W_phi_h``; ``phi = sigmoid(Z)``; ``code = g_self * phi``;
  ``bias = sum_c g_partner,c * code_c`` with fp32 gates)
* sigmoid      ``packages/morphottention/csrc/cuda/morfology/cube.cuh:12-14``; the
  unwired variants HardTanh01 ``clamp((z + 1) / 2, 0, 1)`` and Identity
  (``cube.cuh:15-17,29-35``) and the ``MASK_DIAG`` flag
  (``packages/morphottention/csrc/cuda/utils/declarations.cuh:79-82``), which
  drops key ``j == i``
* scores/mask/online softmax/epilogue
               ``packages/morphottention/csrc/cuda/attention/attention.cu:113-188``
  (``s = (2 S_raw - qb_i - cb_j) * scale * log2e``, causal drop ``k > q``,
  ``lse = m + log2(l)`` in base 2, ``-FLT_MAX`` for an empty row)
* parameters   ``packages/morphottention/torch-ext/morphottention/autograd.py:91-140``
  (``W_phi [D, H*m]``, ``gate_q/gate_k [H, m]``, ``W_V [D, D]``, head ``h``
  owns columns ``h*m..`` and ``h*dv..``; init ``N(0, D^-0.5)`` drawn in fp32 on
  the parameter's device, gates filled with 1; RNG order ``W_phi`` then ``W_V``)
* shape contract ``packages/morphottention/csrc/cuda/attention/attention.cpp:15-57``

Gradients are those of ``torch.autograd`` through this restatement, i.e. the
mathematically complete gradient (the reference CUDA backward drops the
query-side code gradient, ``attention.cu:446-451,472-482``; that defect is not
reproduced).

* soft tropical aggregation (``soft_morph_ref``, ``soft_morph_brute_force``)
               ``packages/morphottention/csrc/cuda/morfology/soft_morph.cuh:10-77``
  (``out = sgn tau ln sum_j exp(sgn (s_ij + V_jc) / tau)`` from the
  ``lse_update`` / ``lse_merge`` / ``lse_finalize`` accumulators, which the
  reference defines but never calls; pinned in ``tests/test_soft_morph_oracle.py``
  against a scalar restatement of those accumulators, the hard max-plus /
  min-plus limit, the large-tau (Hoeffding) bound, erosion-dilation duality,
  the single-key case, the partition of unity of the weights, the
  tau-gradient identity and fp64 gradcheck)

Pinning (all in ``tests/test_oracle.py``): fp64 ``gradcheck``; equivalence with
``F.scaled_dot_product_attention`` on augmented operands; a brute-force
pure-Python loop restatement; the binary-hypercube Hamming closed form; causal
row 0, ``N == 1`` and ``scale == 0`` special cases; score symmetry; head and
batch independence; the identity ``sum_j dS_ij = 0``; committed golden
fixtures. The reference itself ships no tests or golden vectors and cannot run
(CUDA-only), so nothing from it is executed.
"""

from __future__ import annotations

import math

import torch

LOG2E = 1.4426950408889634
FLT_MAX = 3.4028234663852886e38


def init_params(dim: int, num_heads: int, cube_m: int, *, dtype=torch.float32, device="cpu"):
    """Default parameter init of ``MorphoAttention`` (``autograd.py:123-135``).

    ``W_phi`` then ``W_V`` are drawn ``N(0, dim^-0.5)`` in fp32 on ``device``
    from the global generator and cast to ``dtype``; gates are ones.
    """
    std = dim ** -0.5
    head_dim_v = dim // num_heads
    W_phi = torch.empty(dim, num_heads * cube_m, dtype=torch.float32, device=device).normal_(0.0, std)
    W_V = torch.empty(dim, num_heads * head_dim_v, dtype=torch.float32, device=device).normal_(0.0, std)
    gate_q = torch.ones(num_heads, cube_m, dtype=torch.float32, device=device)
    gate_k = torch.ones(num_heads, cube_m, dtype=torch.float32, device=device)
    return W_phi.to(dtype), gate_q.to(dtype), gate_k.to(dtype), W_V.to(dtype)


PROJECTIONS = ("sigmoid", "hardtanh01", "identity")


def cube_project(z, projection: str = "sigmoid"):
    """Cube projection phi(z) (``cube.cuh:12-17``): ``1 / (1 + e^-z)``,
    ``clamp((z + 1) / 2, 0, 1)`` or ``z``."""
    if projection == "sigmoid":
        return torch.sigmoid(z)
    if projection == "hardtanh01":
        return torch.clamp(0.5 * (z + 1.0), 0.0, 1.0)
    if projection == "identity":
        return z
    raise ValueError(f"unknown projection {projection!r}")


def project(x, W_phi, gate_q, gate_k, num_heads: int, cube_m: int, projection: str = "sigmoid"):
    """Per-head soft-hypercube projection (``project.cuh:26-45``, ``cube.cuh:12-17``).

    Returns ``phi, q, k, qb, cb`` with ``phi, q, k`` shaped ``[B, H, N, m]`` and
    ``qb, cb`` shaped ``[B, H, N]``.
    """
    B, N, _ = x.shape
    z = x @ W_phi                                               # [B, N, H*m]
    phi = cube_project(z, projection).view(B, N, num_heads, cube_m).permute(0, 2, 1, 3)
    gq = gate_q.to(phi.dtype)[None, :, None, :]
    gk = gate_k.to(phi.dtype)[None, :, None, :]
    q = gq * phi                                                # code = g_self * phi
    k = gk * phi
    qb = (gk * q).sum(-1)                                       # sum_c g_partner * code
    cb = (gq * k).sum(-1)
    return phi, q, k, qb, cb


def scores(q, k, qb, cb, scale: float):
    """Natural-log scores ``scale * (2 q.k - qb_i - cb_j)`` (``attention.cu:117-125``)."""
    S = q @ k.transpose(-1, -2)
    return scale * (2.0 * S - qb[..., :, None] - cb[..., None, :])


def causal_mask(N: int, device) -> torch.Tensor:
    """True where key ``j > i`` is dropped (``attention.cu:129-130``)."""
    idx = torch.arange(N, device=device)
    return idx[None, :] > idx[:, None]


def drop_mask(N: int, device, causal: bool, mask_diag: bool):
    """True where key ``j`` is dropped from query ``i``'s row: ``j > i`` when
    causal, ``j == i`` with ``MASK_DIAG`` (``attention.cu:126-133``); ``None``
    when nothing is dropped."""
    idx = torch.arange(N, device=device)
    mask = torch.zeros(N, N, dtype=torch.bool, device=device)
    if causal:
        mask |= idx[None, :] > idx[:, None]
    if mask_diag:
        mask |= idx[None, :] == idx[:, None]
    return mask if (causal or mask_diag) else None


def morpho_attention_ref(x, W_phi, gate_q, gate_k, W_V, num_heads: int, cube_m: int, *,
                         scale: float = 1.0, causal: bool = False, return_lse: bool = False,
                         projection: str = "sigmoid", mask_diag: bool = False):
    """Forward of the fused op in the dtype of ``x`` (use fp32 or fp64).

    Returns ``out [B, N, D]`` and, if ``return_lse``, the base-2 row
    log-sum-exp ``lse [B*H, N]`` exactly as ``morphottention::forward`` returns
    it (``attention.cu:173-188``): a row without unmasked keys has ``out = 0``
    and ``lse = -FLT_MAX``.
    """
    B, N, D = x.shape
    H, m = num_heads, cube_m
    dv = W_V.shape[1] // H          # D // H; a head slice of W_V is also accepted
    W_phi = W_phi.to(x.dtype)
    W_V = W_V.to(x.dtype)
    _, q, k, qb, cb = project(x, W_phi, gate_q, gate_k, H, m, projection)
    s = scores(q, k, qb, cb, scale)                             # [B, H, N, N]
    mask = drop_mask(N, x.device, causal, mask_diag)
    empty = None
    if mask is not None:
        s = s.masked_fill(mask, float("-inf"))
        empty = mask.all(dim=-1)                                # rows without keys
        if bool(empty.any()):
            s = s.masked_fill(empty[:, None], 0.0)              # finite, so no NaN reaches autograd
        else:
            empty = None
    lse_nat = torch.logsumexp(s, dim=-1)                        # [B, H, N]
    P = torch.exp(s - lse_nat[..., None])
    if empty is not None:
        P = P.masked_fill(empty[:, None], 0.0)
    V = (x @ W_V).view(B, N, H, dv).permute(0, 2, 1, 3)         # [B, H, N, dv]
    O = P @ V
    out = O.permute(0, 2, 1, 3).reshape(B, N, H * dv)
    if not return_lse:
        return out
    lse = lse_nat * LOG2E
    if empty is not None:
        lse = lse.masked_fill(empty, -FLT_MAX)
    return out, lse.reshape(B * H, N)


def morpho_attention_ref_grads(x, W_phi, gate_q, gate_k, W_V, num_heads: int, cube_m: int, *,
                               scale: float = 1.0, causal: bool = False, dout=None,
                               dtype=torch.float32, batch_chunk: int | None = None,
                               head_chunk: int | None = None, projection: str = "sigmoid",
                               mask_diag: bool = False, heads: tuple[int, int] | None = None):
    """Forward + autograd backward of the restatement, chunked over batch and heads.

    Inputs are upcast to ``dtype``. ``dout`` defaults to ones (i.e. the
    gradient of ``out.sum()``). Returns ``out, lse, (dX, dW_phi, d_gate_q,
    d_gate_k, dW_V)`` in ``dtype``. Chunking bounds the ``[N, N]`` score
    memory and is exact: batch rows never interact, heads only meet in the
    sum of their separate contributions to ``dX``, and the loss
    ``sum(out * dout)`` is a sum over (batch, head) blocks, so the gradients of
    the chunks add up to the full gradient.

    ``heads = (h0, h1)`` evaluates only heads ``h0 .. h1-1``: their output
    columns, ``lse`` rows and parameter-gradient slices are exact, everything
    else is left zero (``dX`` then holds only these heads' share).
    """
    B, N, D = x.shape
    H, m = num_heads, cube_m
    dv = D // H
    bc = batch_chunk or B
    hc = head_chunk or H
    params = [p.detach().to(dtype).clone().requires_grad_(True) for p in (W_phi, gate_q, gate_k, W_V)]
    out = torch.zeros(B, N, D, dtype=dtype, device=x.device)
    lse = torch.zeros(B, H, N, dtype=dtype, device=x.device)
    dX = torch.zeros(B, N, D, dtype=dtype, device=x.device)
    for b0 in range(0, B, bc):
        b1 = min(B, b0 + bc)
        xb = x[b0:b1].detach().to(dtype).clone().requires_grad_(True)
        g_full = torch.ones(b1 - b0, N, D, dtype=dtype, device=x.device) if dout is None \
            else dout[b0:b1].to(dtype)
        hlo, hhi = heads if heads is not None else (0, H)
        for h0 in range(hlo, hhi, hc):
            h1 = min(hhi, h0 + hc)
            o, l = morpho_attention_ref(xb, params[0][:, h0 * m:h1 * m], params[1][h0:h1], params[2][h0:h1],
                                        params[3][:, h0 * dv:h1 * dv], h1 - h0, m,
                                        scale=scale, causal=causal, return_lse=True,
                                        projection=projection, mask_diag=mask_diag)
            o.backward(g_full[:, :, h0 * dv:h1 * dv])
            out[b0:b1, :, h0 * dv:h1 * dv] = o.detach()
            lse[b0:b1, h0:h1] = l.detach().view(b1 - b0, h1 - h0, N)
        dX[b0:b1] = xb.grad.detach()
    grads = (dX, *(p.grad.detach() for p in params))
    return out, lse.reshape(B * H, N), grads


def brute_force_forward(x, W_phi, gate_q, gate_k, W_V, num_heads: int, cube_m: int, *,
                        scale: float = 1.0, causal: bool = False):
    """Pure-Python scalar loops (tiny inputs only), an independent restatement.

    Follows the reference kernel's order of operations: base-2 scores, row max,
    ``exp2``, normalise (``attention.cu:117-188``). Returns nested lists
    ``out[b][i][d]`` and ``lse[b*H + h][i]``.
    """
    B, N, D = x.shape
    H, m = num_heads, cube_m
    dv = D // H
    X = x.tolist()
    Wp = W_phi.tolist()
    Wv = W_V.tolist()
    gq = gate_q.tolist()
    gk = gate_k.tolist()
    out = [[[0.0] * D for _ in range(N)] for _ in range(B)]
    lse = [[0.0] * N for _ in range(B * H)]
    for b in range(B):
        for h in range(H):
            phi = []
            for t in range(N):
                row = []
                for c in range(m):
                    z = sum(X[b][t][d] * Wp[d][h * m + c] for d in range(D))
                    row.append(1.0 / (1.0 + math.exp(-z)))
                phi.append(row)
            qc = [[gq[h][c] * phi[t][c] for c in range(m)] for t in range(N)]
            kc = [[gk[h][c] * phi[t][c] for c in range(m)] for t in range(N)]
            qb = [sum(gk[h][c] * qc[t][c] for c in range(m)) for t in range(N)]
            cb = [sum(gq[h][c] * kc[t][c] for c in range(m)) for t in range(N)]
            V = [[sum(X[b][t][d] * Wv[d][h * dv + e] for d in range(D)) for e in range(dv)] for t in range(N)]
            for i in range(N):
                s2 = []
                for j in range(N):
                    if causal and j > i:
                        continue
                    sraw = sum(qc[i][c] * kc[j][c] for c in range(m))
                    s2.append((j, (2.0 * sraw - qb[i] - cb[j]) * scale * LOG2E))
                mx = max(v for _, v in s2)
                l = sum(2.0 ** (v - mx) for _, v in s2)
                for e in range(dv):
                    acc = sum(2.0 ** (v - mx) * V[j][e] for j, v in s2)
                    out[b][i][h * dv + e] = acc / l
                lse[b * H + h][i] = mx + math.log2(l)
    return out, lse


def sdpa_equivalent(x, W_phi, gate_q, gate_k, W_V, num_heads: int, cube_m: int, *,
                    scale: float = 1.0, causal: bool = False):
    """The attention core written as plain scaled-dot-product attention.

    With ``Q~_i = [2*scale*q_i, 1]`` and ``K~_j = [k_j, -scale*cb_j]`` the score
    ``Q~_i . K~_j = s_ij + scale*qb_i``; the row constant ``scale*qb_i`` cancels
    in the softmax, so ``SDPA(Q~, K~, V, scale=1)`` equals the morpho output.
    Used only to pin ``morpho_attention_ref`` against a library routine.
    """
    import torch.nn.functional as F

    B, N, D = x.shape
    H, m = num_heads, cube_m
    dv = D // H
    _, q, k, qb, cb = project(x, W_phi.to(x.dtype), gate_q, gate_k, H, m)
    ones = torch.ones_like(q[..., :1])
    Qt = torch.cat([2.0 * scale * q, ones], dim=-1)
    Kt = torch.cat([k, (-scale * cb)[..., None]], dim=-1)
    V = (x @ W_V.to(x.dtype)).view(B, N, H, dv).permute(0, 2, 1, 3)
    O = F.scaled_dot_product_attention(Qt, Kt, V, is_causal=causal, scale=1.0)
    return O.permute(0, 2, 1, 3).reshape(B, N, D)


# ---------------------------------------------------------------------------
# Soft tropical aggregation (packages/morphottention/csrc/cuda/morfology/
# soft_morph.cuh:10-77). The reference defines the accumulators but never
# calls them; here they aggregate the values with the morpho scores in place
# of the softmax-weighted sum:
#     out_ic = sgn * tau * ln sum_j exp(sgn * (s_ij + V_jc) / tau)
# sgn = +1 is the soft max-plus product (dilation), sgn = -1 the soft
# min-plus product (erosion); s_ij are the natural-log scores above.


def values(x, W_V, num_heads: int):
    """Per-head values ``V = X W_V,h`` shaped ``[B, H, N, dv]``."""
    B, N, _ = x.shape
    dv = W_V.shape[1] // num_heads
    return (x @ W_V.to(x.dtype)).view(B, N, num_heads, dv).permute(0, 2, 1, 3)


def soft_morph_ref(x, W_phi, gate_q, gate_k, W_V, tau, num_heads: int, cube_m: int, *,
                   scale: float = 1.0, causal: bool = False, sgn: float = 1.0,
                   projection: str = "sigmoid", mask_diag: bool = False, return_zb: bool = False):
    """Soft tropical aggregation in the dtype of ``x`` (fp32 or fp64).

    ``morph_accumulate`` folds ``sgn * (s + v) / tau`` (``soft_morph.cuh:35-38``)
    into a log-sum-exp (``:21-32,41-52``) and ``lse_finalize`` returns
    ``sgn * tau * (m + log l)`` (``:66-69``). ``tau`` is a float or a 0-d
    tensor (differentiable). Returns ``out [B, N, D]`` and, with ``return_zb``,
    the base-2 normaliser ``zb = log2 sum_j 2^(log2e sgn (s_ij + V_jc) / tau)``
    shaped ``[B*H, N, dv]`` (so ``out = sgn tau ln2 zb``). A row without keys
    gives ``out = 0`` and ``zb = -FLT_MAX``.
    """
    B, N, D = x.shape
    H, m = num_heads, cube_m
    W_phi = W_phi.to(x.dtype)
    _, q, k, qb, cb = project(x, W_phi, gate_q, gate_k, H, m, projection)
    s = scores(q, k, qb, cb, scale)                             # [B, H, N, N]
    V = values(x, W_V, H)                                       # [B, H, N, dv]
    dv = V.shape[-1]
    y = sgn * (s[..., :, :, None] + V[..., None, :, :]) / tau   # [B, H, Nq, Nk, dv]
    mask = drop_mask(N, x.device, causal, mask_diag)
    empty = None
    if mask is not None:
        y = y.masked_fill(mask[:, :, None], float("-inf"))
        empty = mask.all(dim=-1)
        if bool(empty.any()):
            y = y.masked_fill(empty[:, None, None], 0.0)
        else:
            empty = None
    lse = torch.logsumexp(y, dim=-2)                            # [B, H, N, dv]
    O = sgn * tau * lse
    if empty is not None:
        O = O.masked_fill(empty[:, None], 0.0)
    out = O.permute(0, 2, 1, 3).reshape(B, N, H * dv)
    if not return_zb:
        return out
    zb = lse * LOG2E
    if empty is not None:
        zb = zb.masked_fill(empty[:, None], -FLT_MAX)
    return out, zb.reshape(B * H, N, dv)


def soft_morph_ref_grads(x, W_phi, gate_q, gate_k, W_V, tau: float, num_heads: int, cube_m: int, *,
                         scale: float = 1.0, causal: bool = False, sgn: float = 1.0, dout=None,
                         dtype=torch.float32, batch_chunk: int | None = None, head_chunk: int | None = None,
                         projection: str = "sigmoid", mask_diag: bool = False):
    """Forward + autograd backward of ``soft_morph_ref``, chunked over batch
    and heads (exact, as in ``morpho_attention_ref_grads``). Returns ``out, zb,
    (dX, dW_phi, d_gate_q, d_gate_k, dW_V, dtau)``."""
    B, N, D = x.shape
    H, m = num_heads, cube_m
    dv = D // H
    bc = batch_chunk or B
    hc = head_chunk or H
    params = [p.detach().to(dtype).clone().requires_grad_(True) for p in (W_phi, gate_q, gate_k, W_V)]
    t = torch.tensor(float(tau), dtype=dtype, device=x.device, requires_grad=True)
    out = torch.empty(B, N, D, dtype=dtype, device=x.device)
    zb = torch.empty(B, H, N, dv, dtype=dtype, device=x.device)
    dX = torch.zeros(B, N, D, dtype=dtype, device=x.device)
    for b0 in range(0, B, bc):
        b1 = min(B, b0 + bc)
        xb = x[b0:b1].detach().to(dtype).clone().requires_grad_(True)
        g_full = torch.ones(b1 - b0, N, D, dtype=dtype, device=x.device) if dout is None \
            else dout[b0:b1].to(dtype)
        for h0 in range(0, H, hc):
            h1 = min(H, h0 + hc)
            o, z = soft_morph_ref(xb, params[0][:, h0 * m:h1 * m], params[1][h0:h1], params[2][h0:h1],
                                  params[3][:, h0 * dv:h1 * dv], t, h1 - h0, m, scale=scale, causal=causal,
                                  sgn=sgn, projection=projection, mask_diag=mask_diag, return_zb=True)
            o.backward(g_full[:, :, h0 * dv:h1 * dv])
            out[b0:b1, :, h0 * dv:h1 * dv] = o.detach()
            zb[b0:b1, h0:h1] = z.detach().view(b1 - b0, h1 - h0, N, dv)
        dX[b0:b1] = xb.grad.detach()
    grads = (dX, *(p.grad.detach() for p in params), t.grad.detach())
    return out, zb.reshape(B * H, N, dv), grads


def soft_morph_brute_force(x, W_phi, gate_q, gate_k, W_V, tau: float, num_heads: int, cube_m: int, *,
                           scale: float = 1.0, causal: bool = False, sgn: float = 1.0, split: int = 2):
    """Pure-Python scalar restatement of the reference accumulators (tiny inputs).

    Per (query, value column): the keys are dealt round-robin into ``split``
    accumulators, each folded key by key with ``lse_update``
    (``soft_morph.cuh:27-31``) of ``sgn (s + v) / tau``; the partial
    accumulators are combined with ``lse_merge`` (``:41-52``), as the
    reference's warp reduction does (``:54-63``), and finished with
    ``lse_finalize`` (``:66-69``). Returns nested lists ``out[b][i][d]``.
    """
    B, N, D = x.shape
    H, m = num_heads, cube_m
    dv = D // H
    X = x.tolist()
    Wp = W_phi.tolist()
    Wv = W_V.tolist()
    gq = gate_q.tolist()
    gk = gate_k.tolist()
    inv_tau = 1.0 / tau

    def update(acc, a):
        mm, ll = acc
        m_new = max(mm, a)
        return (m_new, ll * math.exp(mm - m_new) + math.exp(a - m_new))

    def merge(a, b):
        if a[0] == -math.inf:
            return b
        if b[0] == -math.inf:
            return a
        m_new = max(a[0], b[0])
        return (m_new, a[1] * math.exp(a[0] - m_new) + b[1] * math.exp(b[0] - m_new))

    out = [[[0.0] * D for _ in range(N)] for _ in range(B)]
    for b in range(B):
        for h in range(H):
            phi = [[1.0 / (1.0 + math.exp(-sum(X[b][t][d] * Wp[d][h * m + c] for d in range(D))))
                    for c in range(m)] for t in range(N)]
            qc = [[gq[h][c] * phi[t][c] for c in range(m)] for t in range(N)]
            kc = [[gk[h][c] * phi[t][c] for c in range(m)] for t in range(N)]
            qb = [sum(gk[h][c] * qc[t][c] for c in range(m)) for t in range(N)]
            cb = [sum(gq[h][c] * kc[t][c] for c in range(m)) for t in range(N)]
            V = [[sum(X[b][t][d] * Wv[d][h * dv + e] for d in range(D)) for e in range(dv)] for t in range(N)]
            for i in range(N):
                keys = [j for j in range(N) if not (causal and j > i)]
                s = {j: scale * (2.0 * sum(qc[i][c] * kc[j][c] for c in range(m)) - qb[i] - cb[j]) for j in keys}
                for e in range(dv):
                    parts = [(-math.inf, 0.0) for _ in range(split)]
                    for n, j in enumerate(keys):
                        parts[n % split] = update(parts[n % split], sgn * (s[j] + V[j][e]) * inv_tau)
                    acc = parts[0]
                    for p in parts[1:]:
                        acc = merge(acc, p)
                    out[b][i][h * dv + e] = sgn * tau * (acc[0] + math.log(acc[1]))
    return out

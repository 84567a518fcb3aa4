"""GPU parity of the soft tropical aggregation against the oracle.

``mo.soft_morph_ref`` (pinned in ``tests/test_soft_morph_oracle.py``) in fp32
on the same fp16 inputs is the reference. Bars:

* the output beyond half an fp16 ulp of itself <= 2e-3;
* the fp32 normaliser zb, in output units (tau ln2 |zb - zb_ref|, the error
  of the output before its fp16 rounding), <= 2^-13 max|V| + 1e-4: the
  values carry V_hi + an e4m3 remainder, exact to < 2^-14 |V|, and zb scales
  as 1/tau, so a bar on zb itself would tighten as tau shrinks;
* per gradient tensor max|g - g_ref| / max|g_ref| <= 1e-2; for dtau, which is
  a difference of sums (exactly 0 with one key), the bar is 1e-2 |dtau_ref|
  + 2e-6 sum|dO out| / tau (fp32 cancellation noise of its terms).
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import morpho_oracle as mo

pytestmark = pytest.mark.gpu

FWD_TOL = 2e-3
GRAD_TOL = 1e-2
NAMES = ("dX", "dW_phi", "d_gate_q", "d_gate_k", "dW_V", "dtau")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import morphottention_amd  # noqa: F401
    torch.backends.cuda.matmul.allow_tf32 = False
    yield


def _say(msg):
    print(msg, flush=True)


def _half_ulp(x):
    a = x.abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 11)


def _inputs(B, N, H, m, dv, seed, x_mult=1.0):
    from morphottention_amd import MorphoAttention
    torch.manual_seed(seed)
    mod = MorphoAttention(H * dv, H, m, dtype=torch.float16, device="cpu")
    params = [mod.W_phi.detach(), mod.gate_q.detach(), mod.gate_k.detach(), mod.W_V.detach()]
    g = torch.Generator().manual_seed(seed + 1)
    params[1] = (1.0 + 0.3 * torch.randn(H, m, generator=g)).half()
    params[2] = (1.0 + 0.3 * torch.randn(H, m, generator=g)).half()
    x = (x_mult * torch.randn(B, N, H * dv, generator=g)).half()
    dout = torch.randn(B, N, H * dv, generator=g)
    return x.cuda(), [p.cuda() for p in params], dout.cuda().half()


def _run(x, params, tau, H, m, scale, causal, sgn, dout, projection="sigmoid", mask_diag=False):
    from morphottention_amd import soft_morph_attention
    leaves = [t.detach().clone().requires_grad_(True) for t in (x, *params)]
    t = torch.tensor([tau], dtype=torch.float32, device="cuda", requires_grad=True)
    out = soft_morph_attention(leaves[0], *leaves[1:], t, H, m, scale=scale, causal=causal, erosion=sgn < 0,
                               projection=projection, mask_diag=mask_diag)
    out.backward(dout)
    from morphottention_amd.autograd import variant_bits
    _, zb, _ = torch.ops.morphottention.soft_forward(x, *params, t.detach(), H, m, scale, causal, sgn,
                                                     variant_bits(projection, mask_diag))
    torch.cuda.synchronize()
    return out.detach(), zb, [l.grad for l in leaves] + [t.grad]


def _check(name, out, zb, grads, x, params, tau, H, m, scale, causal, sgn, dout, projection="sigmoid",
           mask_diag=False):
    ref_out, ref_zb, ref_grads = mo.soft_morph_ref_grads(x, *params, tau, H, m, scale=scale, causal=causal, sgn=sgn,
                                                         dout=dout, dtype=torch.float32, projection=projection,
                                                         mask_diag=mask_diag)
    err = (out.float() - ref_out).abs()
    excess = (err - _half_ulp(ref_out)).clamp_min(0).max().item()
    live = ref_zb > -1e38
    zerr = (tau * math.log(2.0) * (zb - ref_zb).abs()).masked_fill(~live, 0.0).max().item()
    vmax = mo.values(x.float(), params[3].float(), H).abs().max().item()
    zbar = 2.0 ** -13 * vmax + 1e-4
    rels = []
    for g, gr in zip(grads, ref_grads):
        gr = gr.float().reshape(g.shape)
        rels.append((g.float() - gr).abs().max().item() / max(gr.abs().max().item(), 1e-30))
    dtau_err = (grads[5].float() - ref_grads[5].float().reshape(grads[5].shape)).abs().item()
    dtau_bar = 1e-2 * ref_grads[5].abs().item() + 2e-6 * (dout.float() * ref_out).abs().sum().item() / tau
    _say(f"[soft] {name}: fwd max-abs {err.max().item():.3e} beyond rounding {excess:.3e} zb (output units) "
         f"{zerr:.2e} (bar {zbar:.2e}) max|out| {ref_out.abs().max().item():.2f} grads "
         + " ".join(f"{n}={r:.2e}" for n, r in zip(NAMES[:5], rels)) + f" dtau {dtau_err:.2e} of {ref_grads[5].abs().item():.2e} (bar {dtau_bar:.2e})")
    assert torch.isfinite(out).all() and all(torch.isfinite(g).all() for g in grads)
    assert excess <= FWD_TOL, f"{name}: forward error beyond fp16 rounding {excess}"
    assert zerr <= zbar, f"{name}: zb error {zerr} in output units"
    for n, r in zip(NAMES[:5], rels):
        assert r <= GRAD_TOL, f"{name}: {n} relative error {r}"
    assert dtau_err <= dtau_bar, f"{name}: dtau error {dtau_err}"


@pytest.mark.parametrize("sgn", [1, -1], ids=["dilation", "erosion"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("m,dv", [(16, 64), (32, 32), (64, 128)])
def test_soft_matches_oracle(m, dv, causal, sgn):
    B, N, H, tau, scale = 2, 100, 2, 0.5, 0.8
    _say(f"[case] soft m={m} dv={dv} causal={causal} sgn={sgn} N={N} tau={tau}")
    x, params, dout = _inputs(B, N, H, m, dv, seed=500 + m + dv)
    out, zb, grads = _run(x, params, tau, H, m, scale, causal, sgn, dout)
    _check(f"m{m} dv{dv} {'causal' if causal else 'full'} sgn{sgn:+d}", out, zb, grads, x, params, tau, H, m, scale,
           causal, sgn, dout)


@pytest.mark.parametrize("tau", [0.05, 4.0])
def test_soft_temperatures(tau):
    B, N, H, m, dv = 2, 129, 2, 16, 64
    _say(f"[case] soft tau={tau} N={N}")
    x, params, dout = _inputs(B, N, H, m, dv, seed=600)
    out, zb, grads = _run(x, params, tau, H, m, 1.0, True, 1, dout)
    _check(f"tau {tau}", out, zb, grads, x, params, tau, H, m, 1.0, True, 1, dout)


@pytest.mark.parametrize("N", [1, 33, 300])
def test_soft_ragged_lengths(N):
    B, H, m, dv = 1, 2, 32, 64
    _say(f"[case] soft N={N}")
    x, params, dout = _inputs(B, N, H, m, dv, seed=700 + N)
    out, zb, grads = _run(x, params, 0.7, H, m, 0.9, False, -1, dout)
    _check(f"N {N}", out, zb, grads, x, params, 0.7, H, m, 0.9, False, -1, dout)


def test_soft_variants_masked_diagonal_and_projection():
    """Causal with the diagonal masked leaves query 0 without keys: out 0,
    zb -FLT_MAX, and no NaN in any gradient; HardTanh01 projection."""
    B, N, H, m, dv = 2, 70, 2, 16, 32
    _say(f"[case] soft mask_diag hardtanh01 N={N}")
    x, params, dout = _inputs(B, N, H, m, dv, seed=800, x_mult=2.0)
    out, zb, grads = _run(x, params, 0.4, H, m, 0.8, True, 1, dout, projection="hardtanh01", mask_diag=True)
    assert bool((out[:, 0] == 0).all()) and bool((zb.view(B, H, N, dv)[:, :, 0] == -mo.FLT_MAX).all())
    _check("mask_diag hardtanh01", out, zb, grads, x, params, 0.4, H, m, 0.8, True, 1, dout,
           projection="hardtanh01", mask_diag=True)


def _soft_sweep_cases(n=20, seed=777):
    """Seeded random cases: batch, length (short and multi-block, ragged),
    heads, cube and head width, causal, dilation / erosion, temperature
    (log-uniform 0.1-4, so some calls take the element-wise fallback),
    scale, projection, masked diagonal (N >= 2) and input magnitude."""
    import numpy as np
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        m = int(rng.choice([16, 32, 64]))
        dv = int(rng.choice([32, 64, 128]))
        H, B = int(rng.integers(1, 4)), int(rng.integers(1, 3))
        N = int(rng.integers(2, 70)) if rng.random() < 0.4 else int(rng.integers(70, 300))
        causal = bool(rng.integers(0, 2))
        sgn = int(rng.choice([1, -1]))
        tau = float(np.round(np.exp(rng.uniform(np.log(0.1), np.log(4.0))), 3))
        scale = float(np.round(rng.uniform(0.3, 1.2), 3))
        projection = str(rng.choice(["sigmoid", "sigmoid", "sigmoid", "hardtanh01"]))
        mask_diag = bool(rng.random() < 0.15)
        x_mult = float(rng.choice([0.5, 1.0, 1.5]))
        cases.append((i, B, N, H, m, dv, causal, sgn, tau, scale, projection, mask_diag, x_mult))
    return cases


SOFT_SWEEP = _soft_sweep_cases()


@pytest.mark.parametrize("case", SOFT_SWEEP, ids=[
    f"s{c[0]}-B{c[1]}-N{c[2]}-H{c[3]}-m{c[4]}-dv{c[5]}-{'causal' if c[6] else 'full'}-"
    f"{'dil' if c[7] > 0 else 'ero'}-tau{c[8]}-{c[10]}{'-md' if c[11] else ''}" for c in SOFT_SWEEP])
def test_soft_random_sweep(case):
    """Each seeded case against the fp32 oracle at the bars above."""
    i, B, N, H, m, dv, causal, sgn, tau, scale, projection, mask_diag, x_mult = case
    _say(f"[case] soft sweep {i}: B={B} N={N} H={H} m={m} dv={dv} causal={causal} sgn={sgn} tau={tau} "
         f"scale={scale} {projection} mask_diag={mask_diag} x_mult={x_mult}")
    x, params, dout = _inputs(B, N, H, m, dv, seed=4000 + i, x_mult=x_mult)
    out, zb, grads = _run(x, params, tau, H, m, scale, causal, sgn, dout, projection=projection, mask_diag=mask_diag)
    _check(f"sweep {i}", out, zb, grads, x, params, tau, H, m, scale, causal, sgn, dout, projection=projection,
           mask_diag=mask_diag)


def test_small_tau_tends_to_the_hard_tropical_product():
    """tau = 1e-3: max_j (s + V) <= out <= max_j (s + V) + tau ln n, up to the
    fp16 rounding of out and the fp16 inputs' projection in fp32."""
    from morphottention_amd import soft_morph_attention
    B, N, H, m, dv, tau = 1, 64, 2, 16, 32, 1e-3
    x, params, _ = _inputs(B, N, H, m, dv, seed=900)
    t = torch.tensor([tau], dtype=torch.float32, device="cuda")
    for sgn in (1, -1):
        out = soft_morph_attention(x, *params, t, H, m, scale=1.0, causal=True, erosion=sgn < 0).float()
        xf = x.float()
        _, q, k, qb, cb = mo.project(xf, params[0].float(), params[1].float(), params[2].float(), H, m)
        s = mo.scores(q, k, qb, cb, 1.0)
        V = mo.values(xf, params[3].float(), H)
        xs = s[..., :, :, None] + V[..., None, :, :]
        keep = ~mo.causal_mask(N, "cuda")[:, :, None]
        hard = (xs.masked_fill(~keep, -math.inf).amax(-2) if sgn > 0 else xs.masked_fill(~keep, math.inf).amin(-2))
        o = out.view(B, N, H, dv).permute(0, 2, 1, 3)
        slack = tau * math.log(N) + _half_ulp(hard).max().item() + 1e-3
        dev = (o - hard).abs().max().item()
        _say(f"[soft] hard limit sgn {sgn:+d}: max |out - hard| {dev:.3e} (slack {slack:.3e})")
        assert dev <= slack


def test_soft_module_trains_tau():
    """SoftMorphAttention: tau is a parameter and receives a finite gradient;
    the output is deterministic across calls."""
    from morphottention_amd import SoftMorphAttention
    torch.manual_seed(3)
    mod = SoftMorphAttention(128, 2, 16, scale=0.7, causal=True, tau=0.6, device="cuda")
    x = torch.randn(2, 50, 128, device="cuda").half()
    out = mod(x)
    out.float().square().mean().backward()
    assert mod.tau.grad is not None and torch.isfinite(mod.tau.grad).all()
    assert torch.equal(out.detach(), mod(x).detach())


def _flag(ws, B, N, D, H, m):
    """The product form's fallback flag in a soft forward workspace: after the
    projection buffers come V's column max and min [B*H, dv] and the row
    references [B*H, N] fp32, each region 256-byte aligned, then the flag."""
    from morphottention_amd import capi
    up = lambda n: (n + 255) // 256 * 256  # noqa: E731
    off = capi.forward_workspace_size(B, N, D, H, m) + 2 * up(B * H * (D // H) * 4) + up(B * H * N * 4)
    return int(ws[off:off + 4].cpu().view(torch.int32).item())


@pytest.mark.parametrize("tau,sgn,causal", [(0.5, 1, True), (0.5, -1, False), (4.0, 1, False), (0.25, -1, True)])
def test_product_form_matches_elementwise_kernels(tau, sgn, causal):
    """Where the product form is exact (its flag stays 0) it gives the
    element-wise kernels' output to within the fp16 rounding of out and the
    normaliser to 2^-16 relative in output units."""
    B, N, H, m, dv = 2, 200, 2, 16, 64
    x, params, _ = _inputs(B, N, H, m, dv, seed=1000)
    t = torch.tensor([tau], dtype=torch.float32, device="cuda")
    fast = torch.ops.morphottention.soft_forward(x, *params, t, H, m, 0.8, causal, sgn, 0)
    exact = torch.ops.morphottention.soft_forward(x, *params, t, H, m, 0.8, causal, sgn, 16)
    torch.cuda.synchronize()
    flag = _flag(fast[2], B, N, H * dv, H, m)
    dz = (tau * math.log(2.0) * (fast[1] - exact[1]).abs()).max().item()
    do = ((fast[0].float() - exact[0].float()).abs() - 2 * _half_ulp(exact[0].float())).max().item()
    _say(f"[soft] product form tau={tau} sgn={sgn:+d} causal={causal}: flag {flag} zb diff (output units) {dz:.2e} "
         f"out diff beyond one ulp {do:.2e}")
    assert flag == 0
    assert dz <= 2.0 ** -16 * (1.0 + exact[0].float().abs().max().item())
    assert do <= 0.0


def test_product_form_falls_back_for_small_tau():
    """tau = 0.02 spreads the exponents beyond the product form's range: the
    flag is raised and the element-wise kernels' result is returned as is."""
    B, N, H, m, dv = 1, 300, 2, 16, 64
    x, params, _ = _inputs(B, N, H, m, dv, seed=1001, x_mult=2.0)
    t = torch.tensor([0.02], dtype=torch.float32, device="cuda")
    fast = torch.ops.morphottention.soft_forward(x, *params, t, H, m, 1.0, True, 1, 0)
    exact = torch.ops.morphottention.soft_forward(x, *params, t, H, m, 1.0, True, 1, 16)
    torch.cuda.synchronize()
    flag = _flag(fast[2], B, N, H * dv, H, m)
    _say(f"[soft] small tau: flag {flag}")
    assert flag == 1
    assert torch.equal(fast[0], exact[0]) and torch.equal(fast[1], exact[1])


def test_exact_switch_gradients_agree():
    """soft_morph_attention(..., exact=True) (element-wise kernels, forward and
    backward) and the default product form give the same gradients to well
    inside the parity bar."""
    from morphottention_amd import soft_morph_attention
    B, N, H, m, dv = 1, 150, 2, 16, 64
    x, params, dout = _inputs(B, N, H, m, dv, seed=1100)
    res = []
    for exact in (False, True):
        leaves = [t.detach().clone().requires_grad_(True) for t in (x, *params)]
        t = torch.tensor([0.6], dtype=torch.float32, device="cuda", requires_grad=True)
        out = soft_morph_attention(leaves[0], *leaves[1:], t, H, m, scale=0.9, causal=True, exact=exact)
        out.backward(dout)
        res.append([g.grad.float() for g in (*leaves, t)])
    rels = [((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item() for a, b in zip(*res)]
    _say("[soft] product form vs element-wise gradients: " + " ".join(f"{n}={r:.2e}" for n, r in zip(NAMES, rels)))
    assert max(rels) <= 2e-3


@pytest.mark.parametrize("sgn", [1, -1], ids=["dilation", "erosion"])
def test_soft_product_form_at_the_benchmarked_head_shape(sgn):
    """The C3 head shape the soft aggregation is benchmarked on (N = 4096,
    cube_m = 16, dv = 64, causal, tau = 0.5; two heads, default init): the
    product form must be the path taken (flag 0), and outputs, zb and every
    gradient including dtau meet the bars against the fp32 oracle (evaluated
    one head at a time: it materialises [N, N, dv] per head)."""
    from morphottention_amd import MorphoAttention
    B, N, H, m, dv, tau, scale = 1, 4096, 2, 16, 64, 0.5, 1.0
    _say(f"[case] soft benchmarked head shape N={N} m={m} dv={dv} sgn={sgn:+d}")
    torch.manual_seed(2)
    mod = MorphoAttention(H * dv, H, m, dtype=torch.float16, device="cpu")
    params = [t.detach().cuda() for t in (mod.W_phi, mod.gate_q, mod.gate_k, mod.W_V)]
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, N, H * dv, generator=g).half().cuda()
    dout = torch.randn(B, N, H * dv, generator=g).half().cuda()
    t = torch.tensor([tau], dtype=torch.float32, device="cuda")
    _, _, ws = torch.ops.morphottention.soft_forward(x, *params, t, H, m, scale, True, sgn, 0)
    torch.cuda.synchronize()
    assert _flag(ws, B, N, H * dv, H, m) == 0, "the product form fell back"
    out, zb, grads = _run(x, params, tau, H, m, scale, True, sgn, dout)
    ref_out, ref_zb, ref_grads = mo.soft_morph_ref_grads(x, *params, tau, H, m, scale=scale, causal=True, sgn=sgn,
                                                         dout=dout, dtype=torch.float32, head_chunk=1)
    err = (out.float() - ref_out).abs()
    excess = (err - _half_ulp(ref_out)).clamp_min(0).max().item()
    zerr = (tau * math.log(2.0) * (zb - ref_zb).abs()).max().item()
    vmax = mo.values(x.float(), params[3].float(), H).abs().max().item()
    zbar = 2.0 ** -13 * vmax + 1e-4
    rels = [(a.float() - b.float().reshape(a.shape)).abs().max().item() / max(b.abs().max().item(), 1e-30)
            for a, b in zip(grads, ref_grads)]
    dtau_bar = 1e-2 * ref_grads[5].abs().item() + 2e-6 * (dout.float() * ref_out).abs().sum().item() / tau
    dtau_err = (grads[5].float() - ref_grads[5].float().reshape(grads[5].shape)).abs().item()
    _say(f"[soft] head shape sgn {sgn:+d}: beyond rounding {excess:.3e} zb {zerr:.2e} (bar {zbar:.2e}) grads "
         + " ".join(f"{n}={r:.2e}" for n, r in zip(NAMES[:5], rels))
         + f" dtau {dtau_err:.2e} of {ref_grads[5].abs().item():.2e} (bar {dtau_bar:.2e})")
    assert excess <= FWD_TOL and zerr <= zbar
    assert all(r <= GRAD_TOL for r in rels[:5]) and dtau_err <= dtau_bar


def test_soft_c_abi_direct_matches_ops():
    """morpho_soft_forward / morpho_soft_backward through ctypes, the C ABI a
    caller without PyTorch binds, on workspaces filled with 0xFF bytes: the
    forward's out and zb equal the torch ops' bit for bit; the gradients agree
    to 1e-3 of each tensor's largest entry (the backward's dq is accumulated
    with fp32 atomics, so their order, not the arithmetic, may differ)."""
    import ctypes
    from morphottention_amd import capi
    L = capi.lib()
    B, N, H, m, dv, scale = 2, 100, 2, 16, 64, 0.8
    D = H * dv
    _say(f"[case] soft C ABI B={B} N={N} H={H} m={m} dv={dv}")
    x, params, dout = _inputs(B, N, H, m, dv, seed=990)
    tau = torch.tensor([0.5], dtype=torch.float32, device="cuda")
    ops = torch.ops.morphottention
    ref_out, ref_zb, ref_ws = ops.soft_forward(x, *params, tau, H, m, scale, True, 1, 0)
    ref_grads = ops.soft_backward(dout, x, *params, tau, ref_zb, ref_ws, H, m, scale, True, 1, 0)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out, zb = torch.empty_like(ref_out), torch.empty_like(ref_zb)
    fbytes = capi.soft_forward_workspace_size(B, N, D, H, m)
    ws = torch.full((fbytes,), 255, dtype=torch.uint8, device="cuda")
    st = L.morpho_soft_forward(*(vp(t) for t in (x, *params, tau, out, zb)), B, N, D, H, m, scale, 1, 1, vp(ws),
                               fbytes, stream)
    assert st == 0, L.morpho_last_error()
    bbytes = capi.soft_backward_workspace_size(B, N, D, H, m, True)
    wb = torch.full((bbytes,), 255, dtype=torch.uint8, device="cuda")
    grads = [torch.empty_like(t) for t in (x, *params, tau)]
    st = L.morpho_soft_backward(*(vp(t) for t in (dout, x, *params, tau, zb, *grads)), B, N, D, H, m, scale, 1, 1,
                                vp(ws), vp(wb), bbytes, stream)
    assert st == 0, L.morpho_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out) and torch.equal(zb, ref_zb)
    for n, g, r in zip(NAMES, grads, ref_grads):
        d = (g.float() - r.float()).abs().max().item() / max(r.float().abs().max().item(), 1e-30)
        assert torch.isfinite(g).all() and d <= 1e-3, f"{n}: C ABI and op differ by {d}"

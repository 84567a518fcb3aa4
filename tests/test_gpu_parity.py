"""GPU parity of the HIP path against the oracle (``oracle/morpho_oracle.py``).

Bars (from the build's north star): forward max-abs error <= 2e-3 and, per
gradient tensor, max|g - g_ref| / max|g_ref| <= 1e-2 versus the fp32 oracle
on the same fp16 inputs. Where the fp16 rounding of the output alone exceeds
2e-3 (large |out|, the wide-cube config), the forward bar is applied to the
error beyond that rounding: |out - ref| - ulp16(ref)/2 <= 2e-3; the plain error
and the rounding floor are printed beside it.
"""

from __future__ import annotations

import ctypes
import glob
import os

import numpy as np
import pytest
import torch

from oracle import morpho_oracle as mo

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FWD_TOL = 2e-3
GRAD_TOL = 1e-2
GRAD_NAMES = ("dX", "dW_phi", "d_gate_q", "d_gate_k", "dW_V")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import morphottention_amd  # noqa: F401  (fails loudly if the build is missing)
    torch.backends.cuda.matmul.allow_tf32 = False
    yield


def _say(msg):
    print(msg, flush=True)


def half_ulp(x: torch.Tensor) -> torch.Tensor:
    """Half a float16 ulp at |x| (normal range), 2^-25 in the subnormal range."""
    a = x.abs().clamp_min(2.0 ** -14)
    e = torch.floor(torch.log2(a))
    return torch.exp2(e - 11)


def run_hip(x, params, H, m, scale, causal, dout):
    from morphottention import morpho_attention  # the reference's import path
    leaves = [t.detach().clone().requires_grad_(True) for t in (x, *params)]
    out = morpho_attention(leaves[0], *leaves[1:], H, m, scale=scale, causal=causal)
    out.backward(dout)
    _, lse = torch.ops.morphottention.forward(x, *params, H, m, scale, causal)
    torch.cuda.synchronize()
    return out.detach(), lse, [t.grad for t in leaves]


# Gradients of the soft-hypercube path. With saturated codes and one-hot
# attention (the wide-cube, 4x-input configuration) they are ~1e-7 of the
# value-path gradients and ill-conditioned: the fp32 oracle itself misses its
# fp64 evaluation by 30-70% there (tests/test_oracle.py::test_fp32_oracle_conditioning).
# In those cases they are checked against an fp64 evaluation of the oracle
# (check_phi_path_fp64) instead of the fp32 one. With a single key they are
# exactly zero, and an absolute bound is used.
PHI_PATH = ("dW_phi", "d_gate_q", "d_gate_k")


def rel_err(g, ref):
    g, ref = g.double(), ref.double()
    return (g - ref).abs().max().item() / max(ref.abs().max().item(), 1e-300)


def check_phi_path_fp64(name, grads, ref32_grads, ref64_grads, heads=None, m=None, bars=None):
    """The HIP soft-hypercube gradients against the fp64 evaluation of the
    oracle, per tensor at GRAD_TOL, or at ``bars[name]`` where given (the fp16
    storage budget of tests/phi_budget.py for the saturated fixture). The fp32
    oracle's own error against fp64 is printed beside. With ``heads = (h0,
    h1)`` only those heads' slices are compared (the fp64 reference was
    evaluated for them alone)."""
    for n in PHI_PATH:
        i = GRAD_NAMES.index(n)
        sl = (slice(None),) if heads is None else (
            (slice(None), slice(heads[0] * m, heads[1] * m)) if n == "dW_phi" else (slice(heads[0], heads[1]),))
        g, r32, r64 = grads[i][sl], ref32_grads[i][sl], ref64_grads[i][sl]
        e_hip, e_32 = rel_err(g, r64), rel_err(r32, r64)
        bar = GRAD_TOL if bars is None else max(GRAD_TOL, bars[n])
        _say(f"[parity-fp64] {name}: {n} HIP {e_hip:.3e} vs fp32 oracle {e_32:.3e} (bar {bar:.3e}, "
             f"max|ref| {r64.abs().max().item():.3e})")
        assert torch.isfinite(g).all()
        assert e_hip <= bar, f"{name}: {n} relative error against fp64 {e_hip} > {bar}"


def check(name, out, lse, grads, ref_out, ref_lse, ref_grads, ill_conditioned=(), zero_phi_path=False):
    ref_out = ref_out.float()
    err = (out.float() - ref_out).abs()
    floor = (ref_out.half().float() - ref_out).abs().max().item()
    excess = (err - half_ulp(ref_out)).clamp_min(0).max().item()
    fwd = err.max().item()
    lse_err = (lse.float() - ref_lse.float()).abs().max().item()
    # The kernel's normaliser sums fp16-rounded weights (each within 2^-12
    # relative), which moves lse by at most log2(1 + 2^-12) = 3.5e-4; the
    # scores themselves are exact to ~2^-22. Bar 1e-3: a key code off by one
    # fp16 ulp (2^-11 relative) moved it by up to 4e-3. lse is also a sum of
    # O(|score|) terms: beyond |lse| ~ 20 (identity projection with wide
    # inputs) fp32 rounding of the projection approaches the bar, so it grows
    # as 5e-5 |lse| there.
    finite = ref_lse.float()[ref_lse.float() > -1e38]
    lse_max = finite.abs().max().item() if finite.numel() else 0.0
    lse_bar = max(1e-3, 5e-5 * lse_max)
    rels = []
    for gname, g, gr in zip(GRAD_NAMES, grads, ref_grads):
        gr = gr.float()
        rels.append((g.float() - gr).abs().max().item() / max(gr.abs().max().item(), 1e-30))
    _say(f"[parity] {name}: fwd max-abs {fwd:.3e} (fp16 floor {floor:.3e}, beyond rounding {excess:.3e}) "
         f"lse {lse_err:.3e} (max |lse| {lse_max:.1f}) grads " + " ".join(f"{n}={r:.2e}" for n, r in zip(GRAD_NAMES, rels)))
    assert torch.isfinite(out).all() and all(torch.isfinite(g).all() for g in grads)
    if floor <= 1e-3:
        assert fwd <= FWD_TOL, f"{name}: forward error {fwd}"
    assert excess <= FWD_TOL, f"{name}: forward error beyond fp16 rounding {excess}"
    assert lse_err <= lse_bar, f"{name}: lse error {lse_err} (max |lse| {lse_max})"
    for n, r, g in zip(GRAD_NAMES, rels, grads):
        if zero_phi_path and n in PHI_PATH:
            scale = ref_grads[GRAD_NAMES.index("dW_V")].abs().max().item()
            assert g.abs().max().item() <= 1e-4 * scale, f"{name}: {n} should vanish"
        elif n not in ill_conditioned:  # those are asserted against fp64 (check_phi_path_fp64)
            assert r <= GRAD_TOL, f"{name}: {n} relative error {r}"
    return fwd, floor, excess, rels


def oracle(x, params, H, m, scale, causal, dout, head_chunk=None):
    N = x.shape[1]
    if head_chunk is None:
        head_chunk = max(1, int(12e9 // (N * N * 4 * 6)))
    return mo.morpho_attention_ref_grads(x, *params, H, m, scale=scale, causal=causal, dout=dout,
                                         dtype=torch.float32, batch_chunk=1, head_chunk=head_chunk)


def make_inputs(B, N, D, H, m, seed, x_mult=1.0, dout_kind="randn", gates=None):
    from morphottention_amd import MorphoAttention
    torch.manual_seed(seed)
    mod = MorphoAttention(D, H, m, dtype=torch.float16, device="cpu")
    params = [mod.W_phi.detach(), mod.gate_q.detach(), mod.gate_k.detach(), mod.W_V.detach()]
    if gates is not None:
        g = torch.Generator().manual_seed(seed + 7)
        params[1] = (gates[0] + gates[1] * torch.randn(H, m, generator=g)).half()
        params[2] = (gates[0] + gates[1] * torch.randn(H, m, generator=g)).half()
    torch.manual_seed(seed)
    x = (x_mult * torch.randn(B, N, D)).half()
    torch.manual_seed(seed + 1000)
    dout = torch.ones(B, N, D) if dout_kind == "ones" else torch.randn(B, N, D)
    dev = "cuda"
    return x.to(dev), [p.to(dev).contiguous() for p in params], dout.half().to(dev)


# ------------------------------------------------------------------ golden fixtures
@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))), ids=os.path.basename)
def test_golden_fixture(path):
    d = np.load(path)
    H, m, scale, causal = int(d["H"]), int(d["cube_m"]), float(d["scale"]), bool(d["causal"])
    t = {k: torch.from_numpy(d[k]).cuda() for k in ("x", "W_phi", "gate_q", "gate_k", "W_V", "dout")}
    params = [t["W_phi"], t["gate_q"], t["gate_k"], t["W_V"]]
    _say(f"[case] golden {os.path.basename(path)} B,N,D={tuple(t['x'].shape)} H={H} m={m} causal={causal}")
    out, lse, grads = run_hip(t["x"], params, H, m, scale, causal, t["dout"])
    ref = [torch.from_numpy(d[k]).cuda() for k in GRAD_NAMES]
    ill = PHI_PATH if "x4" in os.path.basename(path) else ()
    check(os.path.basename(path), out, lse, grads, torch.from_numpy(d["out"]).cuda(),
          torch.from_numpy(d["lse"]).cuda(), ref, ill_conditioned=ill)
    if ill:
        # the fixture holds fp64 gradients. There the phi path's accuracy is
        # set by fp16 storage of dS and dZ (subnormal for the tiny terms of
        # one-hot rows): the bar is 1.5 times the fp64 emulation of exactly
        # those storage points (tests/phi_budget.py; 4.7e-2 for dW_phi, 2.7e-2
        # for the gates), not the fp32 oracle's own error (0.54).
        import phi_budget
        budget = phi_budget.phi_path_budget(path)
        _, _, ref32 = oracle(t["x"], params, H, m, scale, causal, t["dout"])
        check_phi_path_fp64(os.path.basename(path), grads, ref32, ref, bars={n: 1.5 * v for n, v in budget.items()})


# ------------------------------------------------------------------ BASELINE configs
CONFIGS = {
    "C2_B8_N1024_D512_H8_m16": dict(B=8, N=1024, D=512, H=8, m=16, scale=1.0, causal=False, seed=1,
                                    x_mult=1.0, dout_kind="ones"),
    "C3_B4_N4096_D1024_H16_m16_causal": dict(B=4, N=4096, D=1024, H=16, m=16, scale=1.0, causal=True, seed=2,
                                             x_mult=1.0, dout_kind="randn"),
    "C4_B1_N16384_D1024_H16_m32_causal": dict(B=1, N=16384, D=1024, H=16, m=32, scale=0.5, causal=True, seed=3,
                                              x_mult=1.0, dout_kind="randn"),
    "C5_B16_N2048_D2048_H32_m64_x4": dict(B=16, N=2048, D=2048, H=32, m=64, scale=2.0, causal=False, seed=4,
                                          x_mult=4.0, dout_kind="randn", ill=PHI_PATH),
}


@pytest.mark.parametrize("name", list(CONFIGS))
def test_baseline_config(name):
    c = CONFIGS[name]
    _say(f"[case] {name}")
    x, params, dout = make_inputs(c["B"], c["N"], c["D"], c["H"], c["m"], c["seed"], c["x_mult"], c["dout_kind"])
    out, lse, grads = run_hip(x, params, c["H"], c["m"], c["scale"], c["causal"], dout)
    ref_out, ref_lse, ref_grads = oracle(x, params, c["H"], c["m"], c["scale"], c["causal"], dout)
    ill = c.get("ill", ())
    check(name, out, lse, grads, ref_out, ref_lse, ref_grads, ill_conditioned=ill)
    if ill:
        # fp64 oracle on every head, 8 at a time (all batch rows): each
        # chunk's dW_phi columns and gate rows are exact, and each is asserted
        # at GRAD_TOL against them
        for h0 in range(0, c["H"], 8):
            heads = (h0, min(h0 + 8, c["H"]))
            _say(f"[case] {name}: fp64 oracle, heads {heads}")
            _, _, ref64 = mo.morpho_attention_ref_grads(x, *params, c["H"], c["m"], scale=c["scale"],
                                                        causal=c["causal"], dout=dout, dtype=torch.float64,
                                                        batch_chunk=1, head_chunk=8, heads=heads)
            check_phi_path_fp64(f"{name} heads {heads}", grads, ref_grads, ref64, heads=heads, m=c["m"])
            del ref64


# ------------------------------------------------------------------ shape / option matrix
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dv", [32, 64, 128])
@pytest.mark.parametrize("m", [16, 32, 64])
def test_shape_matrix(m, dv, causal):
    B, N, H = 2, 67, 2
    D = H * dv
    _say(f"[case] matrix m={m} dv={dv} causal={causal} B={B} N={N}")
    x, params, dout = make_inputs(B, N, D, H, m, seed=100 + m + dv, gates=(1.0, 0.4))
    out, lse, grads = run_hip(x, params, H, m, 0.8, causal, dout)
    check(f"matrix m{m} dv{dv} {'causal' if causal else 'full'}", out, lse, grads,
          *oracle(x, params, H, m, 0.8, causal, dout))


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("m,dv", [(32, 64), (64, 32), (64, 64)])
def test_eight_wave_backward_key_blocks(m, dv, causal):
    """At m = 32 and 64 (dv <= 64) a backward workgroup has eight waves and
    owns 256 keys, and at m = 32 only four of them have dq tiles. N = 300
    gives two key blocks, the second ragged (44 keys, so waves past N), and
    query steps of 32 that end ragged as well."""
    B, N, H = 2, 300, 2
    _say(f"[case] eight-wave backward m={m} dv={dv} causal={causal} N={N}")
    x, params, dout = make_inputs(B, N, H * dv, H, m, seed=400 + m + dv, gates=(1.0, 0.4))
    out, lse, grads = run_hip(x, params, H, m, 0.8, causal, dout)
    check(f"eight-wave m{m} dv{dv} {'causal' if causal else 'full'}", out, lse, grads,
          *oracle(x, params, H, m, 0.8, causal, dout))


@pytest.mark.parametrize("B,N,D,H,causal", [(7, 1000, 512, 8, False), (7, 1000, 512, 8, True), (3, 300, 256, 4, True)],
                         ids=["T7000-full", "T7000-causal", "320cols-causal"])
def test_projection_tile_128x160(B, N, D, H, causal):
    """Projection tiles of 128 x 160. They are chosen when the 256-row tiles
    fill less than one round of the CUs and 160-column tiles need fewer rounds
    than 128-column ones: T = 7000 with H*M + D = 640 gives 55 row tiles x 4
    (one round) instead of x 5, the last row tile ragged (88 rows). Or when 160
    divides H*M + D and 128 does not: 320 columns, two tiles of 32 code and 128
    value columns each."""
    m = 16
    _say(f"[case] projection 128x160 B={B} N={N} D={D} H={H} causal={causal}")
    x, params, dout = make_inputs(B, N, D, H, m, seed=700 + N + D, gates=(1.0, 0.4))
    out, lse, grads = run_hip(x, params, H, m, 0.8, causal, dout)
    check(f"proj128x160 B{B} N{N} D{D} H{H} {'causal' if causal else 'full'}", out, lse, grads,
          *oracle(x, params, H, m, 0.8, causal, dout))


def test_backward_hi_only_scores_guard():
    """At m = 16 with the sigmoid projection the backward recomputes its
    scores from the fp16 hi codes alone only for heads whose code weights
    sum_c |scale gate_q gate_k| are at most 32; above that from hi and lo
    (an unconditional hi-only backward measured d_gate errors of 1.04e-2
    against fp64 at scale 4 with unit gates). Against the fp64 oracle: scale 4
    with unit gates (sum 64, every head hi / lo) within 3e-3 per tensor; one
    causal launch at scale 1 with heads 0-3 at unit gates (sum 16, hi only,
    within the 1e-2 bar) and heads 4-7 at gates 1.6 (sum 41, hi / lo, within
    3e-3; hi-only there measured up to 6.0e-3)."""
    B, N, D, H, m = 2, 512, 512, 8, 16
    dv = D // H
    x, params, dout = make_inputs(B, N, D, H, m, seed=820)
    gq, gk = params[1].clone(), params[2].clone()
    gq[4:] = 1.6
    gk[4:] = 1.6
    for name, p, scale, causal, hilo_heads in [("scale 4, unit gates", params, 4.0, False, range(H)),
                                               ("mixed heads", [params[0], gq, gk, params[3]], 1.0, True, range(4, H))]:
        _say(f"[case] hi-only guard: {name}")
        out, lse, grads = run_hip(x, p, H, m, scale, causal, dout)
        _, _, r = mo.morpho_attention_ref_grads(x, *p, H, m, scale=scale, causal=causal, dout=dout,
                                                dtype=torch.float64, batch_chunk=1, head_chunk=8)
        _say(f"[parity-fp64] guard {name}: " + " ".join(f"{n}={rel_err(g, ref):.2e}"
                                                       for n, g, ref in zip(GRAD_NAMES, grads, r)))
        for i in range(len(GRAD_NAMES)):
            assert rel_err(grads[i], r[i]) <= GRAD_TOL, f"{name}: {GRAD_NAMES[i]}"
        for h in hilo_heads:  # the heads whose scores must come from hi and lo
            errs = [rel_err(grads[1][:, h * m:(h + 1) * m], r[1][:, h * m:(h + 1) * m]),
                    rel_err(grads[2][h], r[2][h]), rel_err(grads[3][h], r[3][h]),
                    rel_err(grads[4][:, h * dv:(h + 1) * dv], r[4][:, h * dv:(h + 1) * dv])]
            assert max(errs) <= 3e-3, f"{name}: head {h} gradient errors {errs} (hi-only scores?)"


@pytest.mark.parametrize("N", [1, 2, 31, 33, 127, 129, 257])
def test_ragged_lengths(N):
    B, H, m, dv = 3, 4, 16, 64
    _say(f"[case] ragged N={N}")
    x, params, dout = make_inputs(B, N, H * dv, H, m, seed=200 + N)
    for causal in (False, True):
        out, lse, grads = run_hip(x, params, H, m, 1.0, causal, dout)
        check(f"ragged N={N} causal={causal}", out, lse, grads, *oracle(x, params, H, m, 1.0, causal, dout),
              zero_phi_path=(N == 1))


def test_single_key_output_is_v_hi_bitwise():
    """With one key the softmax weight is exactly 1, and the output is
    fp16(V_hi + r 2^-12), r the e4m3 remainder of V - V_hi rounded toward zero:
    it must round back to V_hi bit for bit, the value the backward's dP = dO
    V_hi^T sees. 64 x 1024 values at inputs x3 sweep the remainder over its
    range, both signs, subnormal e4m3 codes included; a remainder rounded to
    nearest instead overshoots the fp16 rounding midpoint for values of V
    near it. V_hi and r are read from the forward workspace (carved as
    capi.hip's carve_proj: qa, ka, then vt [B H, dv, NP] fp16 and vlo
    [B H, NP / 64, dv, 64] e4m3; key 0 sits at column and byte 0)."""
    B, N, D, H, m = 64, 1, 1024, 16, 16
    _say("[case] single key: out == V_hi bitwise")
    x, params, _ = make_inputs(B, N, D, H, m, seed=21, x_mult=3.0)
    out, _, ws = torch.ops.morphottention.forward_train(x, *params, H, m, 1.0, False)
    torch.cuda.synchronize()
    al = lambda n: (n + 255) // 256 * 256  # noqa: E731
    bh, dv, NP, CW = B * H, D // H, 64, 2 * m + 8
    o_vt = 2 * al(bh * N * CW * 2)
    o_vlo = o_vt + al(bh * dv * NP * 2)
    vt = ws[o_vt:o_vt + bh * dv * NP * 2].view(torch.float16).view(bh, dv, NP)[:, :, 0]
    vlo = ws[o_vlo:o_vlo + bh * dv * NP].view(torch.float8_e4m3fn).view(bh, dv, NP)[:, :, 0].float()
    assert (vlo != 0).float().mean().item() > 0.9  # the remainders are carried
    assert (vlo.abs() < 2.0 ** -6).any()  # subnormal e4m3 codes occur
    # the stored pair rounds back to V_hi, and the kernel's output is exactly V_hi
    assert torch.equal((vt.float() + vlo * 2.0 ** -12).half(), vt)
    assert torch.equal(out.view(bh, dv), vt)


@pytest.mark.parametrize("projection", ["sigmoid", "hardtanh01", "identity"])
def test_code_rows_carry_the_codes(projection):
    """Every stored key code pair carries kc = 2 scale log2e G phi: kc_hi +
    kc_lo against c1 G (phi_hi + phi_lo) from the same token's query row,
    relative error <= 2^-18 per code (a consistent pair is exact to ~2^-21).
    Both halves must come from one rounding of the product: evaluated twice
    (once as one rounding of the exact product, once via the fp32 product),
    the two roundings differ at fp16 ties, about 1 code in 16k, and the pair
    then misses kc by a whole fp16 ulp (2^-11), which moves every score
    against that key. 2^20 codes per projection, read from the forward
    workspace (carve_proj: qa, then ka, [B H, N, 2m + 8] fp16)."""
    B, N, H, m, dv = 2, 2048, 4, 64, 64
    scale = 0.9
    from morphottention_amd.autograd import variant_bits
    _say(f"[case] code rows {projection}: B={B} N={N} H={H} m={m}")
    x, params, _ = make_inputs(B, N, H * dv, H, m, seed=33, x_mult=1.5, gates=(1.0, 0.4))
    _, _, ws = torch.ops.morphottention.forward_train(x, *params, H, m, scale, False, variant_bits(projection))
    torch.cuda.synchronize()
    al = lambda n: (n + 255) // 256 * 256  # noqa: E731
    bhn, CW = B * H * N, 2 * m + 8
    qa = ws[:bhn * CW * 2].view(torch.float16).view(B, H, N, CW).double()
    ka = ws[al(bhn * CW * 2):al(bhn * CW * 2) + bhn * CW * 2].view(torch.float16).view(B, H, N, CW).double()
    phi = qa[..., :m] + qa[..., m + 8:]
    G = (params[1].double() * params[2].double())[None, :, None, :]
    kc = 2.0 * scale * 1.4426950408889634 * G * phi
    # bar: 2^-18 relative, with an absolute floor of 2^-20 (fp16 subnormal
    # halves of codes near 0, negligible in an exponent)
    ratio = ((ka[..., :m] + ka[..., m + 8:]) - kc).abs() / (2.0 ** -18 * kc.abs() + 2.0 ** -20)
    worst = ratio.max().item()
    # the key rows' bias pair {b_hi, b_lo} against -log2e scale sum_c G phi,
    # relative to sum_c |G phi| (an fp32 sum: with the Identity projection its
    # terms have both signs and b itself can be small)
    b = -1.4426950408889634 * scale * (G * phi).sum(-1)
    bmag = 1.4426950408889634 * scale * (G * phi).abs().sum(-1)
    bratio = ((ka[..., m] + ka[..., m + 1]) - b).abs() / (2.0 ** -18 * bmag + 2.0 ** -20)
    _say(f"[parity] code rows {projection}: max error of kc_hi + kc_lo {worst:.2e} of the bar, "
         f"codes beyond it: {int((ratio > 1).sum())} of {ratio.numel()}; bias pairs {bratio.max().item():.2e} of it")
    assert worst <= 1.0
    assert bratio.max().item() <= 1.0


def test_scale_zero_is_a_mean():
    B, N, H, m, dv = 2, 96, 2, 16, 64
    x, params, dout = make_inputs(B, N, H * dv, H, m, seed=300)
    out, lse, grads = run_hip(x, params, H, m, 0.0, True, dout)
    check("scale=0 causal", out, lse, grads, *oracle(x, params, H, m, 0.0, True, dout))
    V = x.float() @ params[3].float()
    exp = torch.cumsum(V, dim=1) / torch.arange(1, N + 1, device=V.device)[None, :, None]
    assert (out.float() - exp).abs().max().item() <= FWD_TOL
    assert grads[1].abs().max().item() == 0 and grads[2].abs().max().item() == 0


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("m,dv", [(16, 32), (16, 64), (16, 128), (64, 32), (64, 64), (64, 128)])
def test_value_remainder_is_carried(m, dv, causal):
    """With scale = 0 every weight is exactly 1, so the output is the (prefix)
    mean of V and its only errors are the carried precision of V and the final
    fp16 rounding. V enters as fp16 V_hi plus the remainder V - V_hi in e4m3
    rounded toward zero (relative error < 2^-3 of a term <= 2^-11 |V|), so the
    error beyond half an fp16 ulp of the output is below 2^-14 max|V| in the
    worst case and, on these inputs, at most 2^-18 max|V| (measured). The bar
    is 2^-16 max|V|: with the remainder dropped the excess reaches 2^-13, with
    the remainders paired with the wrong keys of each 64-key tile (visible in
    the masked diagonal tiles) 2^-15 (both measured with the mistake planted
    in a scratch build). The shapes cover the one- and two-block-per-wave
    forwards, the pipelined and one-block tile bodies and the padded
    value-chunk layouts."""
    B, N, H = 2, 200, 2
    x, params, dout = make_inputs(B, N, H * dv, H, m, seed=310 + m + dv)
    from morphottention_amd import morpho_attention
    _say(f"[case] value remainder m={m} dv={dv} causal={causal} N={N}")
    with torch.no_grad():
        out = morpho_attention(x, *params, H, m, scale=0.0, causal=causal).float()
    V = (x.double() @ params[3].double())
    if causal:
        ref = torch.cumsum(V, dim=1) / torch.arange(1, N + 1, device=V.device, dtype=V.dtype)[None, :, None]
    else:
        ref = V.mean(dim=1, keepdim=True).expand_as(V)
    ref = ref.float()
    excess = ((out - ref).abs() - half_ulp(ref)).clamp_min(0).max().item()
    bound = 2.0 ** -16 * V.abs().max().item()
    _say(f"[parity] value remainder m={m} dv={dv} causal={causal}: beyond rounding {excess:.3e} "
         f"(bound {bound:.3e}, max|V| {V.abs().max().item():.2f})")
    assert excess <= bound


def _run_variant(x, params, H, m, scale, causal, dout, projection, mask_diag):
    from morphottention_amd import morpho_attention
    from morphottention_amd.autograd import variant_bits
    leaves = [t.detach().clone().requires_grad_(True) for t in (x, *params)]
    out = morpho_attention(leaves[0], *leaves[1:], H, m, scale=scale, causal=causal, projection=projection,
                           mask_diag=mask_diag)
    out.backward(dout)
    _, lse, _ = torch.ops.morphottention.forward_train(x, *params, H, m, scale, causal,
                                                       variant_bits(projection, mask_diag))
    torch.cuda.synchronize()
    return out.detach(), lse, [t.grad for t in leaves]


# The reference's compile-time variants that it never wires (cube.cuh:9-17,
# declarations.cuh:79-82): HardTanh01 and Identity cube projections, and the
# masked diagonal (which empties query 0's row under causal masking: out 0,
# lse -FLT_MAX). N = 300 spans two forward query blocks and three backward key
# blocks, so unmasked, diagonal and ragged tiles all occur.
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("projection,mask_diag,m,dv", [
    ("hardtanh01", False, 16, 64), ("identity", False, 16, 64), ("hardtanh01", False, 32, 64),
    ("sigmoid", True, 16, 64), ("sigmoid", True, 32, 32), ("sigmoid", True, 64, 128),
    ("identity", True, 16, 32)])
def test_unwired_reference_variants(projection, mask_diag, m, dv, causal):
    B, N, H = 2, 300, 2
    _say(f"[case] variant projection={projection} mask_diag={mask_diag} m={m} dv={dv} causal={causal} N={N}")
    x, params, dout = make_inputs(B, N, H * dv, H, m, seed=1000 + m + dv, x_mult=2.0)
    out, lse, grads = _run_variant(x, params, H, m, 0.7, causal, dout, projection, mask_diag)
    ref = mo.morpho_attention_ref_grads(x, *params, H, m, scale=0.7, causal=causal, dout=dout,
                                        dtype=torch.float32, projection=projection, mask_diag=mask_diag)
    check(f"variant {projection} mask_diag={mask_diag} m={m} dv={dv} causal={causal}", out, lse, grads, *ref)
    if causal and mask_diag:
        assert bool((out[:, 0] == 0).all()) and bool((lse[:, 0] == -3.4028234663852886e38).all())


@pytest.mark.parametrize("causal", [False, True])
def test_exact_max_path_with_large_signed_gates(causal):
    """Gates large and of both signs make the closed-form score bound loose,
    which routes rows through the exact two-pass maximum."""
    B, N, H, m, dv = 2, 200, 2, 32, 64
    x, params, dout = make_inputs(B, N, H * dv, H, m, seed=400, gates=(0.0, 3.0))
    out, lse, grads = run_hip(x, params, H, m, 1.0, causal, dout)
    check(f"signed gates causal={causal}", out, lse, grads, *oracle(x, params, H, m, 1.0, causal, dout))


def _sweep_cases(n=40, seed=20251):
    """Seeded random cases over everything the op accepts at small sizes:
    batch, length (short and multi-block, ragged), heads, cube width, head
    width, causal, projection, masked diagonal, deterministic mode, scale,
    gates and input magnitude. Kept where the fp32 oracle is a sound judge of
    the code-path gradients: scale <= 1 at m = 64, inputs <= 1.5 N(0,1), the
    Identity projection at m <= 32 and scale <= 0.7 (its codes are unbounded)."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        m = int(rng.choice([16, 32, 64]))
        dv = int(rng.choice([32, 64, 128]))
        H, B = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        N = int(rng.integers(2, 70)) if rng.random() < 0.4 else int(rng.integers(70, 420))
        causal = bool(rng.integers(0, 2))
        projection = str(rng.choice(["sigmoid", "sigmoid", "sigmoid", "sigmoid", "hardtanh01", "identity"]))
        if projection == "identity" and m == 64:
            projection = "sigmoid"
        mask_diag = bool(rng.random() < 0.2)
        det = bool(rng.random() < 0.25)
        scale = float(np.round(rng.uniform(0.2, 1.0 if m == 64 else 1.5), 3))
        if projection == "identity":
            scale = min(scale, 0.7)
        gates = (float(rng.choice([0.5, 1.0, 1.5])), float(rng.choice([0.0, 0.3])))
        x_mult = float(rng.choice([0.5, 1.0, 1.5]))
        cases.append((i, B, N, H, m, dv, causal, projection, mask_diag, det, scale, gates, x_mult))
    return cases


SWEEP = _sweep_cases()


@pytest.mark.parametrize("case", SWEEP, ids=[
    f"s{c[0]}-B{c[1]}-N{c[2]}-H{c[3]}-m{c[4]}-dv{c[5]}-{'causal' if c[6] else 'full'}-{c[7]}"
    f"{'-md' if c[8] else ''}{'-det' if c[9] else ''}" for c in SWEEP])
def test_random_sweep(case):
    """Each seeded case against the fp32 oracle at the north star's bars."""
    from morphottention_amd.autograd import variant_bits
    i, B, N, H, m, dv, causal, projection, mask_diag, det, scale, gates, x_mult = case
    _say(f"[case] sweep {i}: B={B} N={N} H={H} m={m} dv={dv} causal={causal} {projection} mask_diag={mask_diag} "
         f"det={det} scale={scale} gates={gates} x_mult={x_mult}")
    x, params, dout = make_inputs(B, N, H * dv, H, m, seed=3000 + i, x_mult=x_mult, gates=gates)
    out, grads = _run_det(x, params, H, m, scale, causal, dout, projection, mask_diag, det)
    _, lse, _ = torch.ops.morphottention.forward_train(x, *params, H, m, scale, causal,
                                                       variant_bits(projection, mask_diag, det))
    ref = mo.morpho_attention_ref_grads(x, *params, H, m, scale=scale, causal=causal, dout=dout,
                                        dtype=torch.float32, projection=projection, mask_diag=mask_diag)
    check(f"sweep {i}", out, lse, grads, *ref)


@pytest.mark.parametrize("projection", ["sigmoid", "hardtanh01"])
def test_causal_rows_ignore_later_tokens(projection):
    """Causal: out and lse of rows < n0 are bit-identical when the inputs of
    tokens >= n0 change (perturbed by 2 N(0,1)), for cut points inside a
    32-row block, at a 64-key tile edge and past the first 256-query
    workgroup. (The exact-max path, which the Identity projection and the
    masked diagonal take, is decided per workgroup, so there a later row can
    change an earlier row's rounding; those are excluded.)"""
    from morphottention_amd.autograd import variant_bits
    B, N, H, m, dv = 2, 700, 2, 16, 64
    _say(f"[case] causality {projection} B={B} N={N}")
    x, params, _ = make_inputs(B, N, H * dv, H, m, seed=950, x_mult=1.5, gates=(1.5, 0.3))
    vb = variant_bits(projection)
    out, lse, _ = torch.ops.morphottention.forward_train(x, *params, H, m, 1.0, True, vb)
    g = torch.Generator(device="cuda").manual_seed(951)
    for n0 in (44, 64, 300):
        x2 = x.clone()
        x2[:, n0:] = (x2[:, n0:].float() + 2.0 * torch.randn(x2[:, n0:].shape, device="cuda", generator=g)).half()
        out2, lse2, _ = torch.ops.morphottention.forward_train(x2, *params, H, m, 1.0, True, vb)
        assert torch.equal(out2[:, :n0], out[:, :n0]), f"n0={n0}: an earlier row's output changed"
        assert torch.equal(lse2.view(B * H, N)[:, :n0], lse.view(B * H, N)[:, :n0]), f"n0={n0}: lse changed"
        assert not torch.equal(out2[:, n0:], out[:, n0:])


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_forward_is_batch_and_head_equivariant(causal):
    """Permuting the batch permutes out and lse; permuting the heads (the
    column blocks of W_phi and W_V and the rows of the gates) permutes the
    output's head columns and lse's head rows. Every (batch, head) problem is
    computed by the same code whatever workgroup, XCD or projection tile
    column it lands on, so both hold bit for bit."""
    B, N, H, m, dv = 3, 300, 4, 32, 64
    _say(f"[case] equivariance causal={causal}")
    x, params, _ = make_inputs(B, N, H * dv, H, m, seed=960, gates=(1.0, 0.4))
    W_phi, gq, gk, W_V = params
    out, lse = torch.ops.morphottention.forward(x, *params, H, m, 0.9, causal)
    pb = torch.tensor([2, 0, 1], device="cuda")
    out_b, lse_b = torch.ops.morphottention.forward(x[pb].contiguous(), *params, H, m, 0.9, causal)
    assert torch.equal(out_b, out[pb])
    assert torch.equal(lse_b.view(B, H, N), lse.view(B, H, N)[pb])
    ph = torch.tensor([3, 1, 0, 2], device="cuda")
    cols = lambda w, width: w.view(w.shape[0], H, width)[:, ph].reshape(w.shape[0], H * width).contiguous()  # noqa: E731
    params_h = [cols(W_phi, m), gq[ph].contiguous(), gk[ph].contiguous(), cols(W_V, dv)]
    out_h, lse_h = torch.ops.morphottention.forward(x, *params_h, H, m, 0.9, causal)
    assert torch.equal(out_h.view(B, N, H, dv), out.view(B, N, H, dv)[:, :, ph])
    assert torch.equal(lse_h.view(B, H, N), lse.view(B, H, N)[:, ph])


def test_gate_gradients_share_one_factor():
    """Kernel outputs obey d_gate_q * gate_q == d_gate_k * gate_k (same dG)."""
    B, N, H, m, dv = 2, 160, 2, 16, 64
    x, params, dout = make_inputs(B, N, H * dv, H, m, seed=500, gates=(1.0, 0.5))
    _, _, grads = run_hip(x, params, H, m, 1.0, True, dout)
    a = grads[2].float() * params[1].float()
    b = grads[3].float() * params[2].float()
    assert (a - b).abs().max().item() <= 2e-2 * a.abs().max().item()


def test_reference_backward_op_recomputes_projection():
    """torch.ops.morphottention.backward (reference schema, no saved
    projection) agrees with the workspace-carrying backward_train."""
    B, N, H, m, dv = 2, 300, 4, 16, 64
    x, params, dout = make_inputs(B, N, H * dv, H, m, seed=600)
    ops = torch.ops.morphottention
    out, lse, ws = ops.forward_train(x, *params, H, m, 1.0, True)
    out2, lse2 = ops.forward(x, *params, H, m, 1.0, True)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    g1 = ops.backward_train(dout, x, *params, out, lse, ws, H, m, 1.0, True)
    g2 = ops.backward(dout, x, *params, out, lse, H, m, 1.0, True)
    for a, b in zip(g1, g2):
        assert (a.float() - b.float()).abs().max().item() <= 1e-3 * max(1.0, a.float().abs().max().item())


def test_forward_is_deterministic():
    B, N, H, m, dv = 2, 513, 4, 32, 64
    x, params, _ = make_inputs(B, N, H * dv, H, m, seed=700)
    a = torch.ops.morphottention.forward(x, *params, H, m, 1.0, False)
    b = torch.ops.morphottention.forward(x, *params, H, m, 1.0, False)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_backward_run_to_run_variation_is_rounding_only():
    """The backward is not bitwise reproducible: dq and the dS row sums are fp32
    atomics from the key-block workgroups, whose order varies. Two runs on the
    same inputs must differ by at most two fp16 ulps per gradient element (the
    fp32 order noise can move an fp16 rounding), with identical forward outputs."""
    B, N, H, m, dv = 2, 1000, 4, 16, 64
    x, params, dout = make_inputs(B, N, H * dv, H, m, seed=710)
    runs = [run_hip(x, params, H, m, 1.0, True, dout) for _ in range(3)]
    for out, lse, grads in runs[1:]:
        assert torch.equal(out, runs[0][0]) and torch.equal(lse, runs[0][1])
        for n, g, g0 in zip(GRAD_NAMES, grads, runs[0][2]):
            a, b = g.float(), g0.float()
            ulp = torch.exp2(torch.floor(torch.log2(torch.maximum(a.abs(), b.abs()).clamp_min(2.0 ** -14))) - 10)
            diff = (a - b).abs()
            _say(f"[determinism] {n}: {int((diff > 0).sum())} of {diff.numel()} elements differ, "
                 f"max {(diff / ulp).max().item():.1f} fp16 ulp")
            assert bool((diff <= 2 * ulp).all()), f"{n}: run-to-run difference beyond two fp16 ulps"


def _run_det(x, params, H, m, scale, causal, dout, projection, mask_diag, deterministic):
    from morphottention_amd import morpho_attention
    leaves = [t.detach().clone().requires_grad_(True) for t in (x, *params)]
    out = morpho_attention(leaves[0], *leaves[1:], H, m, scale=scale, causal=causal, projection=projection,
                           mask_diag=mask_diag, deterministic=deterministic)
    out.backward(dout)
    torch.cuda.synchronize()
    return out.detach(), [t.grad for t in leaves]


# (B, N, H, m, dv, causal, projection, mask_diag): the attn_bwd configurations
# (4 waves / 128 keys at m = 16 and at m = 64 with dv = 128, 8 waves / 256 keys
# at m = 32, 64 with dv <= 64), hi-only and hi/lo scores, steps with and without
# flagged rows (the diagonal kept: only rows with most weight there carry a
# row sum; masked: every row), ragged N and a single key block.
DET_CASES = [
    (2, 1000, 4, 16, 64, True, "sigmoid", False),
    (2, 777, 4, 32, 64, False, "sigmoid", False),
    (1, 600, 2, 64, 128, True, "sigmoid", True),
    (2, 300, 2, 16, 32, False, "hardtanh01", True),
    (3, 33, 2, 64, 32, True, "sigmoid", False),
]


@pytest.mark.parametrize("B,N,H,m,dv,causal,projection,mask_diag", DET_CASES,
                         ids=[f"N{c[1]}-m{c[3]}-dv{c[4]}-{'causal' if c[5] else 'full'}-{c[6]}{'-md' if c[7] else ''}"
                              for c in DET_CASES])
def test_deterministic_backward_is_bitwise_reproducible(B, N, H, m, dv, causal, projection, mask_diag):
    """MORPHO_MODE_DETERMINISTIC: three backward runs give the same bits; the
    gradients meet the oracle bars, and differ from the atomic backward's only
    by the order of the fp32 sums (<= 1e-3 of each tensor's largest entry)."""
    from morphottention_amd.autograd import variant_bits
    _say(f"[case] deterministic B={B} N={N} H={H} m={m} dv={dv} causal={causal} {projection} mask_diag={mask_diag}")
    x, params, dout = make_inputs(B, N, H * dv, H, m, seed=720 + m + dv + N, x_mult=1.5)
    runs = [_run_det(x, params, H, m, 0.8, causal, dout, projection, mask_diag, True) for _ in range(3)]
    for out, grads in runs[1:]:
        assert torch.equal(out, runs[0][0])
        for n, g, g0 in zip(GRAD_NAMES, grads, runs[0][1]):
            assert torch.equal(g, g0), f"{n}: deterministic backward differs between runs"
    out, grads = runs[0]
    _, atomic = _run_det(x, params, H, m, 0.8, causal, dout, projection, mask_diag, False)
    for n, g, ga in zip(GRAD_NAMES, grads, atomic):
        d = (g.float() - ga.float()).abs().max().item() / max(ga.float().abs().max().item(), 1e-30)
        _say(f"[determinism] {n}: deterministic vs atomic {d:.2e} of max")
        assert d <= 1e-3, f"{n}: deterministic and atomic backward differ by {d}"
    _, lse, _ = torch.ops.morphottention.forward_train(x, *params, H, m, 0.8, causal,
                                                       variant_bits(projection, mask_diag, True))
    ref = mo.morpho_attention_ref_grads(x, *params, H, m, scale=0.8, causal=causal, dout=dout,
                                        dtype=torch.float32, projection=projection, mask_diag=mask_diag)
    check(f"deterministic N={N} m={m} dv={dv} causal={causal} {projection} mask_diag={mask_diag}", out, lse, grads,
          *ref)


def test_deterministic_c_abi_overwrites_every_partial():
    """Through the C ABI with mode MORPHO_MODE_CAUSAL | MORPHO_MODE_DETERMINISTIC:
    a workspace filled with 0x00 and one filled with 0xFF (NaN floats) give the
    same bits, equal to the autograd path's, so every partial the reduction
    reads was written by this call; the size query with the mode bits is what
    the call requires."""
    from morphottention_amd import capi
    from morphottention_amd.autograd import variant_bits
    L = capi.lib()
    B, N, H, m, dv = 2, 333, 2, 16, 64
    D = H * dv
    mode = 1 | 32
    x, params, dout = make_inputs(B, N, D, H, m, seed=820)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = torch.empty_like(x)
    lse = torch.empty(B * H, N, dtype=torch.float32, device="cuda")
    fbytes = capi.forward_workspace_size(B, N, D, H, m)
    fws = torch.empty(fbytes, dtype=torch.uint8, device="cuda")
    st = L.morpho_forward(*(vp(t) for t in (x, *params)), vp(out), vp(lse), B, N, D, H, m, 1.0, mode, vp(fws),
                          fbytes, stream)
    assert st == 0, L.morpho_last_error()
    bbytes = capi.backward_workspace_size(B, N, D, H, m, True, mode)
    assert bbytes > capi.backward_workspace_size(B, N, D, H, m, True)
    results = []
    for fill in (0x00, 0xFF):
        bws = torch.full((bbytes,), fill, dtype=torch.uint8, device="cuda")
        grads = [torch.empty_like(t) for t in (x, *params)]
        st = L.morpho_backward(vp(dout), *(vp(t) for t in (x, *params)), vp(out), vp(lse), *(vp(g) for g in grads),
                               B, N, D, H, m, 1.0, mode, vp(fws), vp(bws), bbytes, stream)
        assert st == 0, L.morpho_last_error()
        torch.cuda.synchronize()
        assert all(torch.isfinite(g).all() for g in grads)
        results.append(grads)
    short = L.morpho_backward(vp(dout), *(vp(t) for t in (x, *params)), vp(out), vp(lse), *(vp(g) for g in results[0]),
                              B, N, D, H, m, 1.0, mode, vp(fws), vp(bws), bbytes - 1, stream)
    assert short == 3 and b"backward workspace" in L.morpho_last_error()
    _, auto = _run_det(x, params, H, m, 1.0, True, dout, "sigmoid", False, True)
    for n, a, b, c in zip(GRAD_NAMES, *results, auto):
        assert torch.equal(a, b), f"{n}: stale workspace contents reached the result"
        assert torch.equal(a, c), f"{n}: C ABI and autograd deterministic backward differ"
    ref_out, ref_lse, ref_grads = oracle(x, params, H, m, 1.0, True, dout)
    check("C ABI deterministic backward", out, lse, results[0], ref_out, ref_lse, ref_grads)
    assert variant_bits(deterministic=True) == 32


def test_c_abi_direct_matches_torch_op():
    from morphottention_amd import capi
    L = capi.lib()
    B, N, H, m, dv = 2, 100, 2, 16, 64
    D = H * dv
    x, params, _ = make_inputs(B, N, D, H, m, seed=800)
    ref_out, ref_lse = torch.ops.morphottention.forward(x, *params, H, m, 1.0, True)
    out = torch.empty_like(x)
    lse = torch.empty(B * H, N, dtype=torch.float32, device="cuda")
    nbytes = capi.forward_workspace_size(B, N, D, H, m)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    st = L.morpho_forward(*(ctypes.c_void_p(t.data_ptr()) for t in (x, *params)), ctypes.c_void_p(out.data_ptr()),
                          ctypes.c_void_p(lse.data_ptr()), B, N, D, H, m, 1.0, 1, ctypes.c_void_p(ws.data_ptr()),
                          nbytes, ctypes.c_void_p(stream))
    assert st == 0, L.morpho_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)
    st = L.morpho_forward(*(ctypes.c_void_p(t.data_ptr()) for t in (x, *params)), ctypes.c_void_p(out.data_ptr()),
                          ctypes.c_void_p(lse.data_ptr()), B, N, D, H, m, 1.0, 1, ctypes.c_void_p(ws.data_ptr()),
                          nbytes - 1, ctypes.c_void_p(stream))
    assert st == 3


def _tstat_from_workspace(ws, B, N, D, H, m):
    """The projection's per-query statistics {b, R, gap, t} from the forward
    workspace, whose buffers are laid out one after another in this order,
    each padded to 256 bytes: query rows, key rows [B*H, N, 2m+8] fp16, V_hi^T
    [B*H, dv, NP] fp16, V_lo [B*H, NP, dv] bytes, then the statistics
    [B*H, N] float4."""
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    NP = (N + 63) // 64 * 64
    bhn = B * H * N
    off = 2 * up(bhn * (2 * m + 8) * 2) + up(B * H * NP * (D // H) * 2) + up(B * H * NP * (D // H))
    return ws[off:off + bhn * 16].view(torch.float32).view(B * H, N, 4)


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_fixed_reference_band(causal):
    """Rows whose closed-form bound gap U - t_ii lies in (15, 25] use the
    reference R = U - 15 > t_ii: the row's largest weight may then be as small
    as 2^-10 and the smaller weights reach fp16's subnormal range. Wide cubes
    at scale 2 with unit-variance inputs put most rows in that band; the
    statistics the forward used are read back to show it is reached."""
    B, N, H, m, dv = 1, 4096, 4, 64, 64
    D = H * dv
    _say(f"[case] fixed-reference band m={m} scale=2 N={N} causal={causal}")
    x, params, dout = make_inputs(B, N, D, H, m, seed=1200 + int(causal))
    _, _, ws = torch.ops.morphottention.forward_train(x, *params, H, m, 2.0, causal, 0)
    ts = _tstat_from_workspace(ws, B, N, D, H, m)
    gap = ts[..., 2]
    in_band = ((gap > 15) & (gap <= 25)).float().mean().item()
    # the statistics are the closed form: b and t_ii from the fp32 oracle's projection
    phi, q, k, qb, cb = mo.project(x.float(), params[0].float(), params[1].float(), params[2].float(), H, m)
    b_ref = (-mo.LOG2E * 2.0 * qb).reshape(B * H, N)
    assert (ts[..., 0] - b_ref).abs().max().item() <= 1e-3 * max(1.0, b_ref.abs().max().item())
    _say(f"[parity] band: {100 * in_band:.1f}% of rows with 15 < gap <= 25, max gap {gap.max().item():.1f}")
    assert in_band >= 0.25, f"only {in_band:.3f} of the rows are in the band"
    out, lse, grads = run_hip(x, params, H, m, 2.0, causal, dout)
    check(f"band causal={causal}", out, lse, grads, *oracle(x, params, H, m, 2.0, causal, dout))


@pytest.mark.parametrize("with_fwd_ws", [True, False], ids=["fwd-workspace", "recompute"])
def test_c_abi_backward_matches_oracle(with_fwd_ws):
    """morpho_backward called through ctypes (the boundary a non-Python caller
    binds), with the forward's workspace and with NULL (projection recomputed)."""
    from morphottention_amd import capi
    L = capi.lib()
    B, N, H, m, dv = 2, 150, 2, 32, 64
    D = H * dv
    causal = 1
    x, params, dout = make_inputs(B, N, D, H, m, seed=810, gates=(1.0, 0.3))
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = torch.empty_like(x)
    lse = torch.empty(B * H, N, dtype=torch.float32, device="cuda")
    fbytes = capi.forward_workspace_size(B, N, D, H, m)
    fws = torch.empty(fbytes, dtype=torch.uint8, device="cuda")
    st = L.morpho_forward(*(vp(t) for t in (x, *params)), vp(out), vp(lse), B, N, D, H, m, 1.0, causal, vp(fws),
                          fbytes, stream)
    assert st == 0, L.morpho_last_error()
    grads = [torch.empty_like(t) for t in (x, *params)]
    bbytes = L.morpho_backward_workspace_size(B, N, D, H, m, 1 if with_fwd_ws else 0)
    bws = torch.empty(bbytes, dtype=torch.uint8, device="cuda")
    st = L.morpho_backward(vp(dout), *(vp(t) for t in (x, *params)), vp(out), vp(lse), *(vp(g) for g in grads),
                           B, N, D, H, m, 1.0, causal, vp(fws) if with_fwd_ws else None, vp(bws), bbytes, stream)
    assert st == 0, L.morpho_last_error()
    torch.cuda.synchronize()
    ref_out, ref_lse, ref_grads = oracle(x, params, H, m, 1.0, bool(causal), dout)
    check(f"C ABI backward ({'forward workspace' if with_fwd_ws else 'recomputed projection'})", out, lse, grads,
          ref_out, ref_lse, ref_grads)
    # a workspace one byte short is refused before anything is launched
    st = L.morpho_backward(vp(dout), *(vp(t) for t in (x, *params)), vp(out), vp(lse), *(vp(g) for g in grads),
                           B, N, D, H, m, 1.0, causal, vp(fws) if with_fwd_ws else None, vp(bws), bbytes - 1, stream)
    assert st == 3


def test_error_messages():
    ops = torch.ops.morphottention
    x, params, _ = make_inputs(1, 16, 128, 2, 16, seed=900)
    with pytest.raises(RuntimeError, match="X must be float16"):
        ops.forward(x.float(), *params, 2, 16, 1.0, False)
    with pytest.raises(RuntimeError, match="W_phi must be contiguous"):
        ops.forward(x, params[0].t().contiguous().t(), *params[1:], 2, 16, 1.0, False)
    with pytest.raises(RuntimeError, match=r"W_phi must be \[D, H\*cube_m\]"):
        ops.forward(x, params[0][:, :16].contiguous(), *params[1:], 2, 16, 1.0, False)
    with pytest.raises(RuntimeError, match="D must be divisible by H"):
        ops.forward(x, *params, 3, 16, 1.0, False)
    with pytest.raises(RuntimeError, match=r"unsupported\): cube_m must be 16, 32 or 64 \(got 24\)"):
        W = torch.zeros(128, 48, dtype=torch.float16, device="cuda")
        g = torch.ones(2, 24, dtype=torch.float16, device="cuda")
        ops.forward(x, W, g, g, params[3], 2, 24, 1.0, False)
    # a workspace size of 0 carries the ABI's own reason
    with pytest.raises(RuntimeError, match=r"forward failed \(invalid argument\): Invalid dimensions"):
        ops.forward(x[:0].contiguous(), *params, 2, 16, 1.0, False)
    with pytest.raises(RuntimeError, match=r"backward failed \(unsupported\): head_dim_v = D / H must be"):
        xb = torch.zeros(1, 16, 96, dtype=torch.float16, device="cuda")
        Wp = torch.zeros(96, 32, dtype=torch.float16, device="cuda")
        gg = torch.ones(2, 16, dtype=torch.float16, device="cuda")
        Wv = torch.zeros(96, 96, dtype=torch.float16, device="cuda")
        lse = torch.zeros(2, 16, dtype=torch.float32, device="cuda")
        ops.backward(xb, xb, Wp, gg, gg, Wv, xb, lse, 2, 16, 1.0, False)

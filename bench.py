"""Benchmark of the MI355X morpho-attention hot path (one GPU).

A step is one forward + backward of ``MorphoAttentionFunction`` (the drop-in
autograd bridge) over one synthetic batch already resident in HBM. The default
workload is BASELINE configs[2] (B=4, N=4096, D=1024, H=16, cube_m=16,
causal, fp16), the configuration the headline metric is quoted on.

Prints ONE JSON line on stdout; diagnostics go to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

CONFIGS = {
    # name: B, N, D, H, m, scale, causal, seed, x_mult
    "C2": (8, 1024, 512, 8, 16, 1.0, False, 1, 1.0),
    "C3": (4, 4096, 1024, 16, 16, 1.0, True, 2, 1.0),
    "C4": (1, 16384, 1024, 16, 32, 0.5, True, 3, 1.0),
    "C5": (16, 2048, 2048, 32, 64, 2.0, False, 4, 4.0),
}
PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
# the kernel whose roofline the line reports (the longest of a step at every GPU config)
DOMINANT = "attn_bwd"
PEAK_HBM_GBS = 8000.0
# v_exp_f32 at quarter rate: 256 CUs x 16 lanes/clk x 2.4 GHz (a conservative transcendental bound)
PEAK_EXP_PER_S = 9.8e12
# the CPU reference configuration, timed in every run
C1 = (2, 128, 256, 8, 16, 1.0, False, 0, 1.0)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def pairs(B, N, H, causal):
    return B * H * (N * (N + 1) // 2 if causal else N * N)


def kernel_flops(name, B, N, D, H, m, causal):
    """Algorithmic FLOPs of one launch of each library kernel."""
    T, dv, HM = B * N, D // H, H * m
    P = pairs(B, N, H, causal)
    return {
        "proj_fwd": 2.0 * T * D * (HM + D),
        "attn_fwd": 2.0 * P * (m + dv),
        "attn_bwd": 2.0 * P * (3 * m + 2 * dv),
        "bwd_gemm": 4.0 * T * (HM + D) * D,  # dX and [dW_phi | dW_V] in one launch
    }.get(name)


def step_flops(B, N, D, H, m, causal):
    T, dv, HM = B * N, D // H, H * m
    P = pairs(B, N, H, causal)
    f_fwd = 2.0 * T * D * (HM + D) + 2.0 * P * (m + dv)
    f_bwd = 4.0 * T * D * (HM + D) + 2.0 * P * (3 * m + 2 * dv)
    return f_fwd, f_bwd


def compulsory_bytes(B, N, D, H, m):
    """HBM bytes the step cannot avoid: fwd reads X and the weights and writes
    out and lse; bwd reads dO, X, out, lse and the weights and writes dX and
    the weight gradients (fp16 tensors, fp32 lse)."""
    x = B * N * D * 2
    wts = (D * H * m + D * D + 2 * H * m) * 2
    lse = B * H * N * 4
    fwd = x + wts + x + lse
    bwd = 3 * x + lse + wts + x + wts
    return fwd, bwd


def roofline_terms(flops, exps, nbytes):
    """Time bounds (ms) of one pass: MFMA, exp2 and HBM; the largest binds."""
    t = {"mfma": flops / (PEAK_FP16_TFLOPS * 1e12) * 1e3, "exp": exps / PEAK_EXP_PER_S * 1e3,
         "hbm": nbytes / (PEAK_HBM_GBS * 1e9) * 1e3}
    bound = max(t, key=t.get)
    return bound, {k: round(v, 4) for k, v in t.items()}


def make_inputs(cfg, device, dtype=torch.float16):
    """Synthetic inputs of a config (BASELINE protocol): default MorphoAttention
    init on the CPU in fp32 then rounded to fp16, x ~ xm N(0,1) and dout ~
    N(0,1) rounded to fp16. ``dtype`` float32 gives the same fp16 values upcast
    (the CPU oracle's inputs), on the CPU."""
    from morphottention_amd import MorphoAttention
    B, N, D, H, m, scale, causal, seed, xm = cfg
    torch.manual_seed(seed)
    mod = MorphoAttention(D, H, m, scale=scale, causal=causal, dtype=torch.float16, device="cpu")
    params = [p.detach().to(dtype).to(device).requires_grad_(True)
              for p in (mod.W_phi, mod.gate_q, mod.gate_k, mod.W_V)]
    torch.manual_seed(seed)
    x = (xm * torch.randn(B, N, D)).half().to(dtype).to(device).requires_grad_(True)
    torch.manual_seed(seed + 1000)
    dout = torch.randn(B, N, D).half().to(dtype).to(device)
    return x, params, dout


def load_profile(kind, config):
    """A committed rocprofv3 summary (profiles/<kind>_<config>.json), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", f"{kind}_{config}.json")) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def load_traffic(kernel, config):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary
    (profiles/counters_<config>.json: FETCH_SIZE and WRITE_SIZE per dispatch,
    each scaled by the same counter's reading for a plain copy of known size).
    Offline numbers: PMC passes cannot run inside this timed process."""
    data = load_profile("counters", config)
    try:
        # the profiler names the device function, e.g. attn_bwd -> attn_bwd_kernel
        return data["kernels"][f"{kernel}_kernel"]["hbm_bytes_per_launch"]
    except (TypeError, KeyError):
        return None


def load_trace_avg(kernel, config):
    """Mean duration (ms) of `kernel` over the timed steps of the committed
    rocprofv3 kernel trace of this bench command
    (profiles/kernel_trace_<config>.json), or None."""
    data = load_profile("kernel_trace", config)
    try:
        return data["kernels"][f"{kernel}_kernel"]["timed_avg_us"] / 1e3
    except (TypeError, KeyError):
        return None


def _short_kernel_name(name):
    """`morpho::attn_bwd_kernel<...>(...)` or its mangled form -> `attn_bwd_kernel`."""
    if name.startswith("_ZN6morpho"):
        rest = name[len("_ZN6morpho"):]
        n = 0
        while rest and rest[0].isdigit():
            n = 10 * n + int(rest[0])
            rest = rest[1:]
        return rest[:n]
    return name.split("(")[0].split("<")[0].split("::")[-1]


# SQ counters of the PMC passes (rocprofv3 --pmc, one pass each) and how they
# are normalised: per SIMD, per CU or per wave-cycle, with GRBM_GUI_ACTIVE summed
# over the 8 XCDs (kernel cycles = GRBM_GUI_ACTIVE / 8).
PMC_PASSES = [
    "SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_INST_ANY SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU "
    "SQ_INSTS_MFMA SQ_INSTS_LDS GRBM_GUI_ACTIVE",
    "SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_WAIT_INST_LDS "
    "SQ_VALU_MFMA_COEXEC_CYCLES SQ_INSTS_VALU_TRANS_F32 SQ_ACTIVE_INST_ANY GRBM_GUI_ACTIVE",
    "FETCH_SIZE",
    "WRITE_SIZE",
]


def rocprof_commands(config):
    """The profiling commands whose output --summarize condenses (repo root,
    TMPDIR=/tmp; each PMC pass in a process of its own). The kernel trace runs
    the bench command itself (for C3 the driver's exact command), its JSON line
    kept beside the trace so that the HIP-event figure of the same process can
    be set against the tracer's timestamps."""
    cfg = "" if config == "C3" else f" --config {config}"
    kt = (f"rocprofv3 --kernel-trace --stats -f csv -d gpurun_out/prof/kt_{config} -o run -- "
          f"python bench.py --gpus 1 --steps 20 --warmup 5{cfg} > gpurun_out/prof/kt_{config}.json")
    base = f"python bench.py --config {config} --no-cpu-baseline"
    pmc = [f"rocprofv3 --pmc {ctrs} -f csv -d gpurun_out/prof/pmc{i + 1}_{config} -o run -- "
           f"{base} --steps 1 --warmup 1 --timing-steps 1 --calib-copy" for i, ctrs in enumerate(PMC_PASSES)]
    return kt, pmc


def summarize_rocprof(kind, config, src, steps, warmup, traced_json=None):
    """Condense rocprofv3 CSV output into the committed summary
    profiles/<kind>_<config>.(json|md). kind "kernel_trace": `src` is the
    --kernel-trace output directory; per kernel, the mean duration over the
    dispatches of the timed steps (dispatches warmup .. warmup + steps - 1 of
    each kernel, all of which launch once per step). kind "counters": `src` is
    a comma-separated list of --pmc output directories (PMC_PASSES order, the
    last two FETCH_SIZE and WRITE_SIZE with --calib-copy)."""
    import csv
    import glob as _glob
    os.makedirs(os.path.join(ROOT, "profiles"), exist_ok=True)
    if kind == "kernel_trace":
        f = _glob.glob(os.path.join(src, "*kernel_trace.csv"))[0]
        per = {}
        for r in csv.DictReader(open(f)):
            per.setdefault(_short_kernel_name(r["Kernel_Name"]), []).append(
                (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        out = {"config": config, "command": rocprof_commands(config)[0],
               "summary_command": f"python bench.py --config {config} --steps {steps} --warmup {warmup} "
                                  f"--summarize kernel_trace {src}" +
                                  (f" --traced-json {traced_json}" if traced_json else ""),
               "timed_window":
               f"dispatches {warmup}..{warmup + steps - 1} of each kernel", "kernels": {}}
        for k, v in per.items():
            w = v[warmup:warmup + steps]
            if not w:
                continue
            out["kernels"][k] = {"calls": len(v), "timed_avg_us": round(sum(w) / len(w), 2),
                                 "all_avg_us": round(sum(v) / len(v), 2), "min_us": round(min(v), 2),
                                 "max_us": round(max(v), 2), "timed_us": [round(x, 1) for x in w]}
        if traced_json:
            # the traced process's own line: its dominant kernel's HIP-event
            # mean over the same timed launches, against the tracer's
            line = [ln for ln in open(traced_json) if ln.startswith("{")][-1]
            roof = json.loads(line)["roofline"]
            name = f"{roof['kernel']}_kernel"
            tr = out["kernels"][name]["timed_avg_us"]
            ev = roof["avg_ms"] * 1e3
            out["same_process"] = {"kernel": name, "hip_event_avg_us": round(ev, 2), "trace_avg_us": tr,
                                   "trace_over_events": round(tr / ev, 4), "line_frac": roof["frac"],
                                   "line_ms_per_step": json.loads(line)["ms_per_step"]}
    else:
        dirs = src.split(",")
        vals = {}
        for d in dirs:
            f = _glob.glob(os.path.join(d, "*counter_collection.csv"))[0]
            for r in csv.DictReader(open(f)):
                k = _short_kernel_name(r["Kernel_Name"])
                vals.setdefault(k, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
        mean = {k: {c: sum(v) / len(v) for c, v in d.items()} for k, d in vals.items()}
        # the calibration copy is the largest copyBuffer dispatch of the run
        calib = {c: max(v) for c, v in vals.get("__amd_rocclr_copyBuffer", {}).items()}
        copy_kib = 256 * 1024.0
        ff = copy_kib / calib["FETCH_SIZE"] if calib.get("FETCH_SIZE") else None
        wf = copy_kib / calib["WRITE_SIZE"] if calib.get("WRITE_SIZE") else None
        out = {"config": config, "commands": rocprof_commands(config)[1],
               "summary_command": f"python bench.py --config {config} --summarize counters {src}",
               "calibration": {"copy_bytes": 256 << 20, "fetch_factor": ff, "write_factor": wf,
                               "note": "plain 256 MiB device copy (--calib-copy); factor = known KiB / counter KiB"},
               "kernels": {}}
        for k, a in mean.items():
            if not k.endswith("_kernel"):
                continue
            e = {"counters": {c: round(v, 1) for c, v in sorted(a.items())}}
            cyc = a.get("GRBM_GUI_ACTIVE", 0) / 8.0  # per-XCD kernel cycles
            if cyc and "SQ_VALU_MFMA_BUSY_CYCLES" in a:
                e["mfma_busy"] = round(a["SQ_VALU_MFMA_BUSY_CYCLES"] / (1024 * cyc), 4)
            if "SQ_WAVE_CYCLES" in a and "SQ_WAIT_INST_ANY" in a:
                e["wait_inst_any_per_wave_cycle"] = round(a["SQ_WAIT_INST_ANY"] / a["SQ_WAVE_CYCLES"], 4)
                e["wait_inst_lds_per_wave_cycle"] = round(a.get("SQ_WAIT_INST_LDS", 0) / a["SQ_WAVE_CYCLES"], 4)
            if "SQ_INSTS_MFMA" in a and a["SQ_INSTS_MFMA"]:
                e["valu_per_mfma"] = round((a["SQ_INSTS_VALU"] - a["SQ_INSTS_MFMA"]) / a["SQ_INSTS_MFMA"], 2)
            if cyc and "SQ_LDS_IDX_ACTIVE" in a:
                e["lds_active_per_cu_cycle"] = round(a["SQ_LDS_IDX_ACTIVE"] / (256 * cyc), 4)
                e["lds_bank_conflict_per_active"] = round(a["SQ_LDS_BANK_CONFLICT"] / max(a["SQ_LDS_IDX_ACTIVE"], 1), 4)
            if cyc and "SQ_ACTIVE_INST_VALU" in a:
                e["valu_issue_per_simd_cycle"] = round(4 * a["SQ_ACTIVE_INST_VALU"] / (1024 * cyc), 4)
            if ff and "FETCH_SIZE" in a:
                e["hbm_read_bytes"] = int(a["FETCH_SIZE"] * ff * 1024)
            if wf and "WRITE_SIZE" in a:
                e["hbm_write_bytes"] = int(a["WRITE_SIZE"] * wf * 1024)
            if "hbm_read_bytes" in e and "hbm_write_bytes" in e:
                e["hbm_bytes_per_launch"] = e["hbm_read_bytes"] + e["hbm_write_bytes"]
            out["kernels"][k] = e
    path = os.path.join(ROOT, "profiles", f"{kind}_{config}.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    # a readable table beside the JSON
    lines = [f"# rocprofv3 {kind.replace('_', ' ')}, workload {config}", "", "Commands (repo root, TMPDIR=/tmp):", ""]
    cmds = [out["command"]] if kind == "kernel_trace" else out["commands"]
    lines += [f"    {c}" for c in cmds] + [f"    {out['summary_command']}", ""]
    if kind == "kernel_trace":
        sp = out.get("same_process")
        if sp:
            lines += [f"Same process: {sp['kernel']} HIP events (bound to its dispatches, over the timed steps) "
                      f"{sp['hip_event_avg_us']} us, trace {sp['trace_avg_us']} us (trace / events "
                      f"{sp['trace_over_events']}); that line's frac {sp['line_frac']}, ms_per_step "
                      f"{sp['line_ms_per_step']}.", ""]
        lines += [f"Timed window: {out['timed_window']}.", "",
                  "| kernel | calls | timed avg (us) | all avg (us) | min (us) | max (us) |", "|---|---|---|---|---|---|"]
        for k, v in sorted(out["kernels"].items(), key=lambda kv: -kv[1]["timed_avg_us"]):
            lines.append(f"| {k} | {v['calls']} | {v['timed_avg_us']} | {v['all_avg_us']} | {v['min_us']} | {v['max_us']} |")
    else:
        cols = ["mfma_busy", "valu_issue_per_simd_cycle", "valu_per_mfma", "wait_inst_any_per_wave_cycle",
                "wait_inst_lds_per_wave_cycle", "lds_active_per_cu_cycle", "lds_bank_conflict_per_active",
                "hbm_read_bytes", "hbm_write_bytes"]
        lines += ["mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x kernel cycles); valu_issue = 4 "
                  "SQ_ACTIVE_INST_VALU / (1024 x cycles); wait_* = SQ_WAIT_INST_* / SQ_WAVE_CYCLES; lds_active = "
                  "SQ_LDS_IDX_ACTIVE / (256 CUs x cycles); bank conflicts = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE; "
                  "kernel cycles = GRBM_GUI_ACTIVE / 8 XCDs; HBM bytes = FETCH_SIZE / WRITE_SIZE KiB x the copy "
                  f"calibration factors ({out['calibration']['fetch_factor']:.3f}, "
                  f"{out['calibration']['write_factor']:.3f}).", "",
                  "| kernel | " + " | ".join(cols) + " |", "|---" * (len(cols) + 1) + "|"]
        for k, v in out["kernels"].items():
            lines.append(f"| {k} | " + " | ".join(str(v.get(c, "")) for c in cols) + " |")
    with open(path[:-5] + ".md", "w") as f:
        f.write("\n".join(lines) + "\n")
    log(f"wrote {path} and {path[:-5]}.md")


def calib_copy(device, nbytes=256 << 20):
    """One plain device-to-device copy of a known size (PMC calibration)."""
    src = torch.ones(nbytes, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"calibration copy: {nbytes} bytes read, {nbytes} bytes written")
    del src, dst


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _time_cpu(fn, warmup=2, runs=5, budget_s=15.0):
    """Median wall time (s) of fn() after `warmup` untimed calls; at least one
    and at most `runs` timed calls, fewer when the budget is spent."""
    for _ in range(warmup):
        fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < runs:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s:
            break
    return statistics.median(times), len(times)


def cpu_baseline(cfg, name):
    """The reference has no CPU path (its ops are CUDA-only), so the CPU
    baseline is the eager fp32 oracle (oracle/morpho_oracle.py) on the host
    cores, on the same fp16 input values upcast to fp32: configs[0] (C1)
    in full, and a bounded sample of this
    workload, one batch row with all heads and the full sequence. Each: 2
    warm-up calls, then the median of up to 5 timed calls, forward and
    forward + backward."""
    from oracle import morpho_oracle as mo

    def measure(c, rows):
        B, N, D, H, m, scale, causal, seed, xm = c
        x, params, dout = make_inputs(c, "cpu", dtype=torch.float32)
        x, dout = x.detach()[:rows], dout[:rows]
        params = [p.detach() for p in params]
        with torch.no_grad():
            fwd_s, nf = _time_cpu(lambda: mo.morpho_attention_ref(x, *params, H, m, scale=scale, causal=causal))
        step_s, ns = _time_cpu(lambda: mo.morpho_attention_ref_grads(
            x, *params, H, m, scale=scale, causal=causal, dout=dout, dtype=torch.float32, head_chunk=4))
        return {"fwd_ms": round(fwd_s * 1e3, 2), "fwd_bwd_ms": round(step_s * 1e3, 2),
                "tokens_per_s": round(rows * N / step_s, 1), "runs": [nf, ns]}

    c1 = measure(C1, C1[0])
    B, N = cfg[0], cfg[1]
    w = measure(cfg, 1)
    return {
        "value": w["tokens_per_s"], "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
        "sample": f"oracle fp32 fwd+bwd of 1 of {B} batch rows of {name} (N={N}, all heads): "
                  f"{w['fwd_bwd_ms']} ms (fwd {w['fwd_ms']} ms), median of {w['runs'][1]} runs after 2 warm-ups; "
                  f"C1 (B2 N128 D256 H8 m16, full): fwd+bwd {c1['fwd_bwd_ms']} ms, fwd {c1['fwd_ms']} ms; "
                  f"CPU: {cpu_model()}, os.cpu_count()={os.cpu_count()}, torch threads {torch.get_num_threads()}",
        "workload_sample": w,
        "c1": c1,
    }


def bench_layer(args):
    """fwd+bwd of morphottention_amd.layers.MultiHeadSelfAttention on fp32
    activations at a config's shape: the attn-bench caller (fp16 casts around
    the fused op, then the fp32 output projection). One JSON line."""
    from morphottention_amd.layers import MultiHeadSelfAttention
    B, N, D, H, m, scale, causal, seed, xm = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.manual_seed(seed)
    layer = MultiHeadSelfAttention(D, H, cube_m=m, scale=scale, causal=causal).to(dev)
    x = (xm * torch.randn(B, N, D, device=dev)).requires_grad_(True)
    dout = torch.randn(B, N, D, device=dev)
    leaves = [x, *layer.parameters()]

    def step():
        out, _ = layer(x, x, x)
        return torch.autograd.grad(out, leaves, dout)

    for _ in range(args.warmup):
        step()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    f_fwd, f_bwd = step_flops(B, N, D, H, m, causal)
    f_proj = 3 * 2.0 * B * N * D * D  # output projection: forward and both backward products
    log(f"layer step {ms:.4f} ms ({(f_fwd + f_bwd + f_proj) / (ms * 1e-3) / 1e12:.1f} TFLOP/s incl. projection)")
    print(json.dumps({
        "metric": "MultiHeadSelfAttention fwd+bwd tokens/s (attn-bench caller, fp32 activations)",
        "value": round(B * N / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16 attention, fp32 projection", "data": "synthetic",
        "config": {"workload": f"{args.config} shape through MultiHeadSelfAttention", "global_batch": B,
                   "seq_len": N},
        "step_tflops_incl_projection": round((f_fwd + f_bwd + f_proj) / (ms * 1e-3) / 1e12, 1),
    }), flush=True)


def bench_soft(args):
    """fwd+bwd of the soft tropical aggregation (SoftMorphAttentionFunction,
    learnable tau) at a config's shape. Its kernels do one exp2 per (query,
    key, value column): the bound is the exponential unit, reported as
    achieved exponentials per second against the rate measured on the box.
    One JSON line."""
    from morphottention_amd import SoftMorphAttentionFunction, capi
    B, N, D, H, m, scale, causal, seed, xm = CONFIGS[args.config]
    dv = D // H
    dev = torch.device("cuda:0")
    x, params, dout = make_inputs(CONFIGS[args.config], dev)
    tau = torch.full((1,), args.tau, dtype=torch.float32, device=dev, requires_grad=True)
    sgn = -1 if args.erosion else 1
    leaves = [x, *params, tau]

    def step():
        out = SoftMorphAttentionFunction.apply(x, *params, tau, H, m, scale, causal, sgn)
        return torch.autograd.grad(out, leaves, dout)

    for _ in range(args.warmup):
        step()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    capi.timing_enable(True)
    capi.timing_read()
    for _ in range(args.timing_steps):
        step()
    torch.cuda.synchronize()
    recs = capi.timing_read()
    capi.timing_enable(False)
    per = {}
    for name, t in recs:
        per.setdefault(name, []).append(t)
    P = pairs(B, N, H, causal)
    # algorithmic work of the aggregation: the element-wise kernels do one
    # exp2 per (query, key, column); the product form does the same FLOPs as
    # the softmax path (scores and one value product forward; scores, two
    # value products and the code gradients backward)
    work = {"soft_fwd": ("exp", P * dv), "soft_bwd": ("exp", P * dv),
            "soft_fwd_fast": ("mfma", 2.0 * P * (m + dv)), "soft_bwd_fast": ("mfma", 2.0 * P * (3 * m + 2 * dv))}
    kernels = {}
    avgs = {k: sum(v) / len(v) for k, v in per.items()}
    for exact in ("soft_fwd", "soft_bwd"):
        # faster than the exponential unit allows: the product form was exact
        # and the element-wise kernel only read its flag
        if exact in avgs and work[exact][1] / (avgs[exact] * 1e-3) > PEAK_EXP_PER_S:
            work.pop(exact)
    for name, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        avg = sum(v) / len(v)
        kind, amount = work.get(name, (None, None))
        rate = amount / (avg * 1e-3) if amount else None
        kernels[name] = {"avg_ms": round(avg, 5), "kind": kind, "rate": rate and round(rate / 1e12, 3)}
        note = ""
        if kind == "exp":
            note = f"  {rate / 1e12:.2f}e12 exp/s ({rate / PEAK_EXP_PER_S:.1%})"
        elif kind == "mfma":
            note = f"  {rate / 1e12:.1f} TFLOP/s ({rate / 1e12 / PEAK_FP16_TFLOPS:.1%})"
        log(f"  {name:18s} {avg:8.4f} ms" + note)
    log(f"soft step {ms:.4f} ms")
    # the dominant kernel that did the work (an element-wise kernel that found
    # the product form exact only checks its flag)
    dom = max((k for k in per if k in work), key=lambda k: sum(per[k]))
    dom_avg = sum(per[dom]) / len(per[dom])
    kind, amount = work[dom]
    print(json.dumps({
        "metric": "soft tropical aggregation fwd+bwd tokens/s",
        "value": round(B * N / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16 in/out, fp32 exponent arithmetic", "data": "synthetic",
        "config": {"workload": f"{args.config} shape, soft {'erosion' if sgn < 0 else 'dilation'} tau={args.tau}",
                   "global_batch": B, "seq_len": N},
        "roofline": ({"bound": "exp", "kernel": dom, "achieved": round(amount / (dom_avg * 1e-3) / 1e12, 3),
                      "peak": PEAK_EXP_PER_S / 1e12, "unit": "1e12 exp2/s",
                      "frac": round(amount / (dom_avg * 1e-3) / PEAK_EXP_PER_S, 4)} if kind == "exp" else
                     {"bound": "mfma", "kernel": dom, "achieved": round(amount / (dom_avg * 1e-3) / 1e12, 1),
                      "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                      "frac": round(amount / (dom_avg * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4)}),
        "kernels": kernels,
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C3", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--timing-steps", type=int, default=5, help="steps re-run with per-kernel HIP events")
    ap.add_argument("--calib-copy", action="store_true", help="run one 256 MiB copy first (PMC calibration)")
    ap.add_argument("--layer", choices=["mhsa", "soft"], default=None,
                    help="time the attn-bench MultiHeadSelfAttention layer (fp32 in/out), or the soft tropical "
                         "aggregation, instead of the bare op")
    ap.add_argument("--tau", type=float, default=0.5, help="--layer soft: temperature")
    ap.add_argument("--erosion", action="store_true", help="--layer soft: soft min-plus instead of max-plus")
    ap.add_argument("--traced-json", default=None,
                    help="--summarize kernel_trace: the JSON line the traced bench command printed")
    ap.add_argument("--summarize", nargs=2, metavar=("KIND", "SRC"), default=None,
                    help="write profiles/<KIND>_<config>.json from rocprofv3 CSV output: KIND kernel_trace (SRC = "
                         "the --kernel-trace directory of this command) or counters (SRC = comma-separated --pmc "
                         "directories); no GPU work")
    args = ap.parse_args()
    if args.summarize:
        return summarize_rocprof(args.summarize[0], args.config, args.summarize[1], args.steps, args.warmup,
                                 args.traced_json)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; the path is sharded over "
                                   "(batch x head) without collectives"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}))
        sys.exit(1)

    from morphottention_amd import MorphoAttentionFunction, capi

    if args.layer == "soft":
        return bench_soft(args)
    if args.layer:
        return bench_layer(args)
    cfg = CONFIGS[args.config]
    B, N, D, H, m, scale, causal, seed, xm = cfg
    dev = torch.device("cuda:0")
    if args.calib_copy:
        calib_copy(dev)
    x, params, dout = make_inputs(cfg, dev)
    leaves = [x, *params]

    def fwd():
        return MorphoAttentionFunction.apply(x, *params, H, m, scale, causal)

    def step():
        out = fwd()
        return torch.autograd.grad(out, leaves, dout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # --- timed region: exactly K fwd+bwd steps. The dominant kernel carries
    # HIP events bound to its own dispatches (hipExtLaunchKernel on the launch
    # stream), so its average duration comes from these very launches. Only it
    # is timed here: a timed dispatch waits a few microseconds in the queue.
    capi.timing_only(DOMINANT)
    capi.timing_enable(True)
    capi.timing_read()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps
    dom_recs = [t for name, t in capi.timing_read() if name == DOMINANT]
    capi.timing_enable(False)
    capi.timing_only(None)
    assert len(dom_recs) == args.steps, f"{len(dom_recs)} {DOMINANT} launches timed in {args.steps} steps"

    # --- forward only (reported beside)
    with torch.no_grad():
        for _ in range(3):
            fwd()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            fwd()
        e1.record()
        torch.cuda.synchronize()
    ms_fwd = e0.elapsed_time(e1) / args.steps

    # --- every kernel's duration, from HIP events bound to the dispatches of
    # `--timing-steps` further steps (a per-kernel table beside the line)
    capi.timing_enable(True)
    capi.timing_read()
    for _ in range(args.timing_steps):
        step()
    torch.cuda.synchronize()
    recs = capi.timing_read()
    capi.timing_enable(False)

    # --- the same K steps again, after every pass above (about 2K + 8 more
    # steps of load): beside the line, not its value. The driver's window
    # follows W warm-up steps after an idle GPU, while the clock is still
    # settling; this shows the step once it has.
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms_after = e0.elapsed_time(e1) / args.steps
    per = {}
    for name, ms in recs:
        per.setdefault(name, []).append(ms)
    kernels = {}
    for name, v in per.items():
        avg = sum(v) / len(v)
        f = kernel_flops(name, B, N, D, H, m, causal)
        kernels[name] = {"avg_ms": round(avg, 5), "launches_per_step": len(v) / args.timing_steps,
                         "tflops": round(f / (avg * 1e-3) / 1e12, 1) if f else None}
    dominant = DOMINANT
    if per and max(per, key=lambda k: sum(per[k])) != dominant:
        log(f"note: {max(per, key=lambda k: sum(per[k]))} took longer than {dominant} in the timing steps")
    dom_avg = sum(dom_recs) / len(dom_recs)
    dom_flops = kernel_flops(dominant, B, N, D, H, m, causal)
    achieved = dom_flops / (dom_avg * 1e-3) / 1e12
    f_fwd, f_bwd = step_flops(B, N, D, H, m, causal)
    b_fwd, _ = compulsory_bytes(B, N, D, H, m)
    bound, terms = roofline_terms(f_fwd, pairs(B, N, H, causal), b_fwd)
    fwd_roof = {"bound": bound, "terms_ms": terms, "frac": round(terms[bound] / ms_fwd, 4)}
    for k, v in sorted(kernels.items(), key=lambda kv: -kv[1]["avg_ms"]):
        log(f"  {k:18s} {v['avg_ms']:8.4f} ms  x{v['launches_per_step']:.0f}/step  {v['tflops']} TFLOP/s")
    log(f"step {ms_step:.4f} ms  fwd {ms_fwd:.4f} ms  step-level {(f_fwd + f_bwd) / (ms_step * 1e-3) / 1e12:.1f} "
        f"TFLOP/s  (the same steps after the other passes: {ms_after:.4f} ms)")

    log(f"{dominant} over the timed steps: {dom_avg:.4f} ms ({len(dom_recs)} launches, HIP events)")
    roofline = {"bound": "mfma", "kernel": dominant, "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
                "traffic": load_traffic(dominant, args.config),
                "avg_ms": round(dom_avg, 5), "timed_launches": len(dom_recs)}
    trace_ms = load_trace_avg(dominant, args.config)
    if trace_ms:
        # the same kernel's mean over the timed steps of the committed
        # rocprofv3 kernel trace of this command (the tracer's own timestamps)
        roofline["rocprof"] = {"avg_ms": round(trace_ms, 5),
                               "achieved": round(dom_flops / (trace_ms * 1e-3) / 1e12, 2),
                               "frac": round(dom_flops / (trace_ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4)}
    result = {
        "metric": "fwd+bwd ms & tokens/s at B4 N4096 D1024 H16 causal fp16; % of roofline",
        "value": round(B * N / (ms_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (x ~ N(0,1), dout ~ N(0,1), default MorphoAttention init)",
        "config": {"workload": f"{args.config}: B={B} N={N} D={D} H={H} cube_m={m} scale={scale} "
                               f"causal={causal} fwd+bwd", "global_batch": B, "seq_len": N},
        "fwd_ms": round(ms_fwd, 4),
        "fwd_tokens_per_s": round(B * N / (ms_fwd * 1e-3), 1),
        "ms_per_step_after_passes": round(ms_after, 4),
        "step_roofline_frac": round((f_fwd + f_bwd) / 2.5e15 / (ms_step * 1e-3), 4),
        "fwd_roofline": fwd_roof,
        "roofline": roofline,
        "kernels": kernels,
    }
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle on host cores)...")
        result["cpu_baseline"] = cpu_baseline(cfg, args.config)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()

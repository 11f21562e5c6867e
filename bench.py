#!/usr/bin/env python3
"""Benchmark: one layer of GPTQ calibration on one MI355X.

Default workload (the north-star target): a
Qwen3-30B-A3B-shaped MoE layer -- 128 experts, hidden 2048,
moe_intermediate 768, 131072 tokens routed top-8 -- solved end to end:
  per-expert Hessians (gate_up: routed gather of the hidden states, 2048^2;
  down: the experts' SiLU(g)*u inputs, 768^2), damped per-group Cholesky
  inverses, MXFP4 safe-scale-search GPTQ for every routed expert, RTN for
  the 4 unrouted experts (they have no Hessian), and MLX uint32 packing of
  all codes.

--config 1|2|3|5 runs the dense BASELINE configs instead (one Hessian per
distinct input, GPTQ of every matrix in the config's mode, packing):
  1 single Linear [2048,2048] affine 4-bit, 8192 tokens
  2 q_proj [4096,4096] MXFP4 groupwise, 32768 tokens
  3 up [14336,4096] + down [4096,14336] MXFP8 groupwise, 65536 tokens
  5 gate, up [25600,5120] + down [5120,25600] MXFP4 safe search, 524288 tokens

Inputs (hidden states, routing, weights) are synthetic, seeded, and
resident in HBM before the timed region. One step = one layer. The JSON
line reports weight elements solved per second, the dominant kernel against
its roofline, and the CPU oracle (the reference algorithm restated on
torch-CPU) timed on the same workload: in full for configs 1-4, in full
for config 5 but for its down-proj Hessian, which is timed on 65536 of its
524288 tokens and scaled linearly in tokens.

Usage: python bench.py [--config 4] [--gpus 1] [--steps K] [--warmup W] [--cpu-sample] [--cpu-seconds S]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-gptq-mxfp_amd"))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0
PEAK_FP64_TFLOPS = 78.6  # MI355X fp64 (vector and matrix)
MXFP_BYTES_PER_ELEMENT = 2 + 4 + 1 + 1 / 32  # bf16 W in, f32 W_dq + u8 code out, E8M0 scale


def _args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--config", type=int, default=4, choices=(1, 2, 3, 4, 5))
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="time budget of the CPU-oracle sample taken with --cpu-sample; "
                         "0 disables the CPU leg")
    ap.add_argument("--cpu-sample", action="store_true",
                    help="dense configs: time the CPU oracle on a bounded sample of about "
                         "--cpu-seconds and scale it, instead of the whole layer. Without it "
                         "every part is timed in full except a Hessian above 2e14 dense flops "
                         "(config 5's 25600-wide down input, about 8 minutes on the host), "
                         "timed on 65536 tokens and scaled linearly in tokens")
    ap.add_argument("--gemm-ceiling", action="store_true",
                    help="time torch.matmul / torch.bmm in bf16 (hipBLASLt) on a square GEMM and "
                         "on the config-4 gate_up Gram shapes instead of the solve: the vendor "
                         "library's sustained bf16 rate on this box, beside the SYRK's")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="before the steps, run one plain elementwise copy (torch.neg) of this many "
                         "MiB: the reference dispatch that scales rocprofv3 FETCH_SIZE / WRITE_SIZE "
                         "to bytes")
    ap.add_argument("--capture", action="store_true",
                    help="config 4 only: time the routed capture path instead of the solve "
                         "(per-batch RoutedStash.add_routed, plan, one grouped Hessian launch), "
                         "with the reference's per-expert CPU stash path timed beside it")
    ap.add_argument("--audit", action="store_true",
                    help="config 4 only: time the fused artifact range audit over the layer's "
                         "gate_up weights and their MXFP4 RTN codes instead of the solve")
    return ap.parse_args(argv)


def _traffic(name: str, kernel_prefix: str):
    """HBM bytes per launch of a kernel: rocprofv3 FETCH_SIZE + WRITE_SIZE of
    that dispatch, each scaled by what the counter reads for a plain 1 GiB
    copy, as committed under profiles/ (the profiler cannot run inside this
    process). None if absent."""
    p = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        per = json.load(f).get("bytes_per_dispatch", {})
    hits = [v for k, v in per.items() if k.startswith(kernel_prefix)]
    return round(float(max(hits))) if hits else None


def _counter(name: str, kernel_prefix: str, key: str):
    """A per-dispatch rocprofv3 counter figure of a kernel (e.g. its MFMA
    util %) as committed under profiles/<name>_counters.json; None if
    absent."""
    p = os.path.join(ROOT, "profiles", f"{name}_counters.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        per = json.load(f).get("per_dispatch", {})
    hits = [v[key] for k, v in per.items() if k.startswith(kernel_prefix) and key in v]
    return max(hits) if hits else None


def _counters_in_order(name: str, kernel_prefix: str, key: str):
    """The same figure for every distinct dispatch of a kernel, in launch
    order (profiles/<name>_counters.json keeps the first dispatch of each
    grid size, in the order the profiled step launched them)."""
    p = os.path.join(ROOT, "profiles", f"{name}_counters.json")
    if not os.path.exists(p):
        return []
    with open(p) as f:
        per = json.load(f).get("per_dispatch", {})
    return [v[key] for k, v in per.items() if k.startswith(kernel_prefix) and key in v]


def _roofline(kernel, bound, amount, ms, traffic=None):
    """amount: flops (bound "mfma": bf16 MFMA peak; "fp64": fp64 peak) or bytes
    (bound "hbm") per launch."""
    if bound in ("mfma", "fp64"):
        peak = PEAK_BF16_TFLOPS if bound == "mfma" else PEAK_FP64_TFLOPS
        achieved, unit = amount / (ms * 1e-3) / 1e12, "TFLOP/s"
    else:
        achieved, peak, unit = amount / (ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
    return {"kernel": kernel, "bound": bound, "achieved": round(achieved, 1), "peak": peak,
            "unit": unit, "frac": round(achieved / peak, 4), "traffic": traffic,
            "per_launch": amount, "launch_ms": round(ms, 4)}


def _copy_calibration(torch, dev, mib):
    if mib <= 0:
        return
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.neg(src, out=dst)  # reads and writes exactly n*4 bytes
    torch.cuda.synchronize()
    del src, dst


def _events(torch, n):
    """A step's own timing events (steps run back to back, so each needs its own)."""
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def _timed(torch, np, step, n_phase, warmup, steps):
    """Warmup, then exactly `steps` steps between two device synchronizations
    (the host queues step i+1 while the GPU runs step i, as a layer-by-layer
    driver would). Phase times and the per-step median come from each step's
    own events, read after the closing synchronization: a step's first event
    completes when the previous step's work has, so its span is that step's
    time on the GPU."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    phase = np.zeros(n_phase)
    out = None
    all_evs = []
    t0 = time.perf_counter()
    for _ in range(steps):
        out, evs = step()
        all_evs.append(evs)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    per_step = []
    for evs in all_evs:
        phase += [evs[i].elapsed_time(evs[i + 1]) for i in range(n_phase)]
        per_step.append(evs[0].elapsed_time(evs[n_phase]))
    _timed.median_ms = float(np.median(per_step)) if per_step else 0.0
    return out, (t1 - t0) * 1e3 / steps, phase / steps


def _line(args, value, ms_step, config, phases, roofline, cpu, setup_s, extra=None):
    line = {
        "metric": "GPTQ weight-elements solved/s per layer",
        "value": round(value, 1),
        "unit": "elements/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "ms_per_step_median": round(getattr(_timed, "median_ms", ms_step), 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16+fp32",
        "data": "synthetic (seeded hidden states, routing and weights of the config's shapes)",
        "config": config,
        "phases_ms": {k: round(float(v), 3) for k, v in phases.items()},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "setup_s": round(setup_s, 2),
    }
    if extra:
        line.update(extra)
    print(json.dumps(line), flush=True)


# ---------------------------------------------------------------------------
# config 4: routed-expert MoE layer
# ---------------------------------------------------------------------------
def run_moe(args, torch, np) -> int:
    from mlx_gptq import capture, gptq, grid, packing, synth

    dev = torch.device("cuda", 0)
    t_setup = time.perf_counter()
    L = synth.moe_layer(device=dev)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    E, ne = L.experts, L.experts - L.n_empty
    hidden, inter = L.W_gate_up.shape[2], L.W_down.shape[2]
    counts = L.counts()
    assert all(c > 0 for c in counts[:ne]) and all(c == 0 for c in counts[ne:])
    A = L.offsets[-1]
    elements = E * (2 * inter * hidden + hidden * inter)

    H_gu = torch.empty(E, hidden, hidden, dtype=torch.float32, device=dev)
    H_dn = torch.empty(E, inter, inter, dtype=torch.float32, device=dev)
    # Each projection's codes are packed by its solve (packed_out: the
    # solver writes pack_q's words from the codes it holds), so they are not
    # read back from HBM by a separate packing pass.
    # Every step plans its Hessian launches from scratch: a real calibration
    # sees a new routing (new expert offsets) in every layer, so the plan
    # cache of grouped_hessian would miss each time.
    def step():
        evs = _events(torch, 6)
        capture.clear_hessian_plan_cache()
        evs[0].record()
        capture.grouped_hessian(L.X, L.offsets, L.row_index, out=H_gu, validate=False)
        evs[1].record()
        capture.grouped_hessian(L.Y, L.offsets, out=H_dn)
        evs[2].record()
        p_gu = torch.empty(ne, 2 * inter, hidden // 8, dtype=torch.int32, device=dev)
        q_gu, s_gu, _, wq_gu, _ = gptq.solve_gptq(L.W_gate_up[:ne], H_gu[:ne], 4, 32, mode="mxfp4",
                                                  packed_out=p_gu)
        evs[3].record()
        p_dn = torch.empty(ne, hidden, inter // 8, dtype=torch.int32, device=dev)
        q_dn, s_dn, _, wq_dn, _ = gptq.solve_gptq(L.W_down[:ne], H_dn[:ne], 4, 32, mode="mxfp4",
                                                  packed_out=p_dn)
        evs[4].record()
        rq_gu, rs_gu, _, _ = grid.rtn_quantize_mxfp(L.W_gate_up[ne:], "mxfp4")
        rq_dn, rs_dn, _, _ = grid.rtn_quantize_mxfp(L.W_down[ne:], "mxfp4")
        packed = [p_gu, p_dn] + [packing.pack_q(q, 4) for q in (rq_gu, rq_dn)]
        evs[5].record()
        return (q_gu, s_gu, q_dn, s_dn, packed), evs

    _copy_calibration(torch, dev, args.copy_calib_mib)
    out, ms_step, phase = _timed(torch, np, step, 5, args.warmup, args.steps)
    value = elements / (ms_step * 1e-3)
    roofline = _roofline("syrk_kernel (gate_up Hessian, routed gather)", "mfma",
                         A * hidden * (hidden + 1),  # SYRK count N*C*(C+1)
                         float(phase[0]), _traffic("bench_moe_cfg4", "mgq::syrk_kernel<true"))
    cpu = _cpu_baseline_moe(L, ne, out, (H_gu, H_dn)) if args.cpu_seconds > 0 else None
    config = {
        "workload": "cfg4 Qwen3-30B-A3B MoE layer: 128 experts x (gate_up [1536,2048] + down "
                    "[2048,768]), 131072 tokens top-8, MXFP4 safe-scale-search GPTQ, 4 unrouted "
                    "experts RTN, uint32 pack",
        "experts": E, "hidden": hidden, "moe_intermediate": inter, "tokens": L.X.shape[0],
        "top_k": A // L.X.shape[0], "assignments": A, "elements": elements,
    }
    phases = {"hessian_gate_up": phase[0], "hessian_down": phase[1],
              "solve_and_pack_gate_up": phase[2], "solve_and_pack_down": phase[3],
              "rtn_and_pack_unrouted": phase[4]}
    # rocprofv3 MFMA-busy / active cycles of the two SYRK launches and the
    # solver's VALU-busy share. The profiler cannot run inside this process,
    # so these are NOT measured by this run: they are read from the committed
    # per-dispatch counters of an earlier profiled run of this workload.
    counters = {"from_profile": {
        "source": "profiles/bench_moe_cfg4_counters.json (rocprofv3 --pmc of bench.py, an "
                  "earlier run; not measured in this run)",
        "hessian_mfma_util_pct": {
            "gate_up": _counter("bench_moe_cfg4", "mgq::syrk_kernel<true", "mfma_util_pct"),
            "down": _counter("bench_moe_cfg4", "mgq::syrk_kernel<false", "mfma_util_pct")},
        "hessian_clock_ghz": {
            "gate_up": _counter("bench_moe_cfg4", "mgq::syrk_kernel<true", "clock_ghz"),
            "down": _counter("bench_moe_cfg4", "mgq::syrk_kernel<false", "clock_ghz")},
        "solve_valu_busy_pct": _counter("bench_moe_cfg4", "mgq::mxfp_solve_kernel",
                                        "valu_busy_pct"),
        "solve_valu_insts_per_row_group": _counter("bench_moe_cfg4", "mgq::mxfp_solve_kernel",
                                                   "valu_insts_per_lane_item")},
        "hessian_plan": "cold: planned and uploaded inside every timed step (new routing per layer)"}
    # every phase against its own bound: the SYRKs against bf16 MFMA, the
    # solve + pack phases against HBM with their algorithmic bytes (bf16 W in,
    # f32 W_dq + u8 code + E8M0 scale + the packed 4-bit code out)
    el_gu = ne * 2 * inter * hidden
    el_dn = ne * hidden * inter
    per_el = MXFP_BYTES_PER_ELEMENT + 0.5
    counters["phase_rooflines"] = {
        "hessian_gate_up": roofline,
        "hessian_down": _roofline("syrk_kernel (down Hessian, expert rows)", "mfma",
                                  A * inter * (inter + 1), float(phase[1]),
                                  _traffic("bench_moe_cfg4", "mgq::syrk_kernel<false")),
        "solve_and_pack_gate_up": _roofline("MXFP4 safe-search solve + pack (gate_up)", "hbm",
                                            el_gu * per_el, float(phase[2])),
        "solve_and_pack_down": _roofline("MXFP4 safe-search solve + pack (down)", "hbm",
                                         el_dn * per_el, float(phase[3])),
    }
    _line(args, value, ms_step, config, phases, roofline, cpu, setup_s, counters)
    return 0


def run_capture(args, torch, np) -> int:
    """Routed capture of the config-4 layer's gate_up inputs: 64 batches of
    2048 tokens, each stashed once with its top-8 expert ids, then every
    expert's H from one grouped launch. The reference's path (one CPU bf16
    Stash per expert filled with the gathered rows, capture.py:42-50, then
    per-expert fp32 addmm on the GPU, capture.py:68-76) is timed beside it on
    the first batches."""
    from mlx_gptq import capture, synth

    dev = torch.device("cuda", 0)
    t_setup = time.perf_counter()
    L = synth.moe_layer(device=dev)
    E, T = L.experts, L.X.shape[0]
    hidden = L.X.shape[1]
    counts = torch.tensor(L.counts(), device=dev)
    expert_of = torch.repeat_interleave(torch.arange(E, device=dev), counts)
    order = torch.argsort(L.row_index.long(), stable=True)
    top_k = expert_of[order].reshape(T, -1)  # the router's choice per token
    K = top_k.shape[1]
    bt = 2048
    batches = [(a, min(a + bt, T)) for a in range(0, T, bt)]
    H = torch.empty(E, hidden, hidden, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    stash = capture.RoutedStash("gate_up", hidden, E)

    def step():
        evs = _events(torch, 4)
        stash.clear()
        evs[0].record()
        for a, b in batches:
            stash.add_routed(L.X[a:b], top_k[a:b])
        evs[1].record()
        stash.plan()
        evs[2].record()
        stash.hessians(out=H)
        evs[3].record()
        return H, evs

    out, ms_step, phase = _timed(torch, np, step, 3, args.warmup, args.steps)
    A = T * K
    # parity with the solve path's Hessians (same rows, other order)
    H_ref = capture.grouped_hessian(L.X, L.offsets, L.row_index)
    rel = float(((out - H_ref).norm() / H_ref.norm()).item())
    roofline = _roofline("syrk_kernel (gate_up Hessian, routed gather)", "mfma", A * hidden * (hidden + 1),
                         float(phase[2]), _traffic("bench_moe_cfg4", "mgq::syrk_kernel<true"))
    # the reference's per-expert stash path on the first batches (skipped
    # with --cpu-seconds 0)
    nb = min(len(batches), 4)
    ref = None
    if args.cpu_seconds > 0:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        stashes = [[] for _ in range(E)]
        for a, b in batches[:nb]:
            xb, tb = L.X[a:b], top_k[a:b]
            for e in range(E):
                tok = torch.nonzero((tb == e).any(dim=1)).flatten()
                if tok.numel():
                    stashes[e].append(xb[tok].to("cpu", torch.bfloat16))
        t1 = time.perf_counter()
        for e in range(E):
            Hm = torch.zeros(hidden, hidden, dtype=torch.float32, device=dev)
            for c in stashes[e]:
                x = c.to(dev, torch.float32, non_blocking=True)
                Hm.addmm_(x.T, x)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        a_ref = sum(b - a for a, b in batches[:nb]) * K
        ref = {"value": round(a_ref / (t2 - t0), 1), "unit": "assignments/s",
               "kind": "reference path (torch, GPU + host copies)",
               "sample": f"first {nb} of {len(batches)} batches: per-expert gather + copy to CPU bf16 "
                         f"{(t1 - t0) * 1e3:.1f} ms, per-expert fp32 addmm Hessians "
                         f"{(t2 - t1) * 1e3:.1f} ms",
               "cores": torch.get_num_threads()}
    line = {
        "metric": "routed-capture assignments/s (stash + plan + grouped Hessian)",
        "value": round(A / (ms_step * 1e-3), 1),
        "unit": "assignments/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16+fp32",
        "data": "synthetic (config-4 hidden states and top-8 routing)",
        "config": {"workload": f"cfg4 gate_up capture: {T} tokens in {len(batches)} batches of {bt}, "
                               f"top-{K} of {E} experts, hidden {hidden}",
                   "assignments": A},
        "phases_ms": {"add_routed": round(float(phase[0]), 3), "plan": round(float(phase[1]), 3),
                      "hessian": round(float(phase[2]), 3)},
        "roofline": roofline,
        "rel_frobenius_vs_solve_path_hessians": rel,
        "reference_path": ref,
        "setup_s": round(setup_s, 2),
    }
    print(json.dumps(line), flush=True)
    return 0


def run_audit(args, torch, np) -> int:
    """Range audit (validate_artifacts.py:21-55) of the config-4 gate_up
    weights: bf16 [128 x 1536, 2048] source, u8 codes, E8M0 scales. One fused
    launch reads 2 + 1 + 1/32 bytes per element."""
    from mlx_gptq import grid, synth, validate_artifacts

    dev = torch.device("cuda", 0)
    t_setup = time.perf_counter()
    L = synth.moe_layer(device=dev)
    src = L.W_gate_up.reshape(-1, L.W_gate_up.shape[-1])
    q, sb, _, _ = grid.rtn_quantize_mxfp(src, "mxfp4")
    del L
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    def step():
        evs = _events(torch, 2)
        evs[0].record()
        st = validate_artifacts.range_audit(src, q, sb, None, "mxfp4", 32)
        evs[1].record()
        return st, evs

    st, ms_step, phase = _timed(torch, np, step, 1, args.warmup, args.steps)
    n = src.numel()
    nbytes = n * (2 + 1) + n // 32
    roofline = _roofline("range_audit_kernel", "hbm", nbytes, float(phase[0]))
    cpu = None
    if args.cpu_seconds > 0:
        sys.path.insert(0, ROOT)
        from oracle import validate_ref

        info = _cpu_setup(torch)
        rows = max(1, min(src.shape[0], 8192))
        s_c, q_c, b_c = src[:rows].cpu(), q[:rows].cpu(), sb[:rows].cpu()
        t0 = time.perf_counter()
        want = validate_ref.range_audit(s_c, q_c, b_c, None, "mxfp4", 32)
        t1 = time.perf_counter()
        got = validate_artifacts.range_audit(src[:rows], q[:rows], sb[:rows], None, "mxfp4", 32)
        cpu = {"value": round(rows * src.shape[1] / (t1 - t0), 1), "unit": "elements/s",
               **info, "kind": "port",
               "sample": f"first {rows} rows: torch-CPU restatement of validate_artifacts.py:15-55, "
                         f"{(t1 - t0) * 1e3:.1f} ms", "matches_gpu": got == want}
    line = {
        "metric": "artifact range-audit elements/s", "value": round(n / (ms_step * 1e-3), 1),
        "unit": "elements/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 source, u8 codes, f64 ratios",
        "data": "synthetic (config-4 gate_up weights and their MXFP4 RTN codes)",
        "config": {"workload": f"cfg4 gate_up range audit: [{src.shape[0]}, {src.shape[1]}] bf16",
                   "elements": n},
        "phases_ms": {"range_audit": round(float(phase[0]), 3)},
        "roofline": roofline, "cpu_baseline": cpu, "result": st, "setup_s": round(setup_s, 2),
    }
    print(json.dumps(line), flush=True)
    return 0


def _cpu_setup(torch) -> dict:
    """CPU leg threads and host description: one thread per core of this
    process's affinity (the reference's CPU solve runs multi-threaded
    torch), capped at the host share the box grants (OMP_NUM_THREADS); the
    CPU model and the torch build."""
    aff = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or aff
    threads = max(1, min(aff, share))
    torch.set_num_threads(threads)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")),
                         model)
    except OSError:
        pass
    return {"cores": threads, "affinity_cores": aff, "cpu_model": model,
            "torch": torch.__version__, "mkl": bool(torch.backends.mkl.is_available())}


def _cpu_baseline_moe(L, ne, gpu_out, H_gpu):
    """The reference's path on the host CPU (the oracle: a torch-CPU
    restatement of capture.py:68-76, gptq.py and packing.py), in the shape
    sequential.py:536-626 runs it, timed in full on the whole layer:
    per-expert fp32 addmm Hessians of every routed expert, then ONE stacked
    solve_gptq over all routed experts per projection (the reference's span
    holds all of them at its default 16 GiB budget), RTN for the unrouted
    experts and numpy packing. The stacked solves are given the GPU's
    Hessians, so both sides solve identical inputs and their codes can be
    compared element for element."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import gptq_ref, grid_ref, hessian_ref, packing_ref

    info = _cpu_setup(torch)
    hidden, inter = L.W_gate_up.shape[2], L.W_down.shape[2]
    q_gu, _, q_dn, _, _ = gpu_out
    H_gu, H_dn = H_gpu
    A = L.offsets[ne]
    # 1. Hessians of every routed expert (rows gathered on the host first,
    #    as the reference's CPU stashes hold them)
    hess_s = 0.0
    for e in range(ne):
        a, b = L.offsets[e], L.offsets[e + 1]
        xs = L.X.index_select(0, L.row_index[a:b].long()).cpu()
        ys = L.Y[a:b].cpu()
        t = time.perf_counter()
        hessian_ref.stash_hessian([xs], hidden)
        hessian_ref.stash_hessian([ys], inter)
        hess_s += time.perf_counter() - t
    # 2. one stacked MXFP4 safe-search solve per projection over all routed experts
    solve_s, agree_n, agree_d = 0.0, 0, 0
    for W, H, q_g in ((L.W_gate_up, H_gu, q_gu), (L.W_down, H_dn, q_dn)):
        Wc = W[:ne].cpu()
        Hc = H[:ne].cpu()
        t = time.perf_counter()
        rq, _, _, _, _ = gptq_ref.solve_gptq(Wc, Hc, 4, 32, mode="mxfp4")
        solve_s += time.perf_counter() - t
        agree_n += int((q_g.cpu() == rq).sum())
        agree_d += rq.numel()
        del Wc, Hc, rq
    # 3. RTN of the unrouted experts and numpy packing of every code tensor
    t = time.perf_counter()
    rq_g, _, _, _ = grid_ref.rtn_quantize_mxfp(L.W_gate_up[ne:].cpu().float(), "mxfp4")
    rq_d, _, _, _ = grid_ref.rtn_quantize_mxfp(L.W_down[ne:].cpu().float(), "mxfp4")
    for qq in (q_gu.cpu().numpy(), q_dn.cpu().numpy(), rq_g.numpy(), rq_d.numpy()):
        packing_ref.pack_q(qq, 4)
    tail_s = time.perf_counter() - t
    total = hess_s + solve_s + tail_s
    elements = L.W_gate_up.numel() + L.W_down.numel()
    return {
        "value": round(elements / total, 1),
        "unit": "elements/s",
        **info,
        "kind": "port",
        "extrapolated": False,
        "seconds": {"hessians": round(hess_s, 2), "solve": round(solve_s, 2),
                    "rtn_and_pack": round(tail_s, 2), "layer": round(total, 2)},
        "sample": (f"the whole layer, nothing extrapolated: fp32 addmm Hessians (65536-row "
                   f"chunks) of all {ne} routed experts ({A} assignments, gate_up and down "
                   f"inputs); one stacked MXFP4 safe-search solve_gptq of all {ne} routed experts "
                   f"per projection, on the GPU's Hessians; RTN of the {L.experts - ne} unrouted "
                   f"experts and numpy pack_q of every code tensor"),
        "code_agreement_with_gpu": round(agree_n / max(agree_d, 1), 6),
    }


# ---------------------------------------------------------------------------
# configs 1, 2, 3, 5: dense layers
# ---------------------------------------------------------------------------
def run_dense(args, torch, np) -> int:
    from mlx_gptq import capture, gptq, synth

    dev = torch.device("cuda", 0)
    t_setup = time.perf_counter()
    L = synth.dense_config(args.config, device=dev)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    keys = list(L.inputs)
    # the drop-in path: each input's rows in a capture.Stash (the reference's
    # per-matrix stash, capture.py:33-79), its H from Stash.hessian
    stashes = {}
    for k in keys:
        st = capture.Stash(k, L.inputs[k].shape[1])
        st.add(L.inputs[k])
        L.inputs[k] = st.chunks[0]  # the stash's copy; the generated one is freed
        stashes[k] = st
    torch.cuda.synchronize()
    n_ev = len(keys) + len(L.mats)
    # each matrix's codes packed by its solve (packed_out), as pack_q would
    def packed_shape(m):
        B_, R_, C_ = m.W.shape
        return (B_, R_, C_ * m.pack_bits // 32)

    def step():
        evs = _events(torch, n_ev + 1)
        i = 0
        evs[i].record()
        Hs = {}
        for k in keys:
            Hs[k] = stashes[k].hessian(dev).unsqueeze(0)
            i += 1
            evs[i].record()
        res, packed = [], []
        for m in L.mats:
            packed.append(torch.empty(packed_shape(m), dtype=torch.int32, device=dev))
            res.append(gptq.solve_gptq(m.W, Hs[m.inp], **m.solve, packed_out=packed[-1]))
            i += 1
            evs[i].record()
        return (res, packed, Hs), evs

    _copy_calibration(torch, dev, args.copy_calib_mib)
    out, ms_step, phase = _timed(torch, np, step, n_ev, args.warmup, args.steps)
    elements = L.elements
    value = elements / (ms_step * 1e-3)
    phases, rooflines = {}, {}
    tag = f"bench_dense_cfg{args.config}"
    for i, k in enumerate(keys):
        N, C = L.inputs[k].shape
        phases[f"hessian_{k}"] = phase[i]
        rooflines[f"hessian_{k}"] = _roofline(f"syrk_kernel (Hessian of '{k}', [{N}x{C}])", "mfma",
                                              N * C * (C + 1), float(phase[i]))
    for j, m in enumerate(L.mats):
        ms = float(phase[len(keys) + j])
        phases[f"solve_and_pack_{m.name}"] = ms
        n = int(m.W.numel())
        if m.solve["mode"] == "affine":
            # O(C^3) work: the fp64 factor + inverse (2C^3/3 algorithmic, potrf +
            # trtri) and the deferred fp32 update 2 R sum_blocks bs (C - i2),
            # framed against the fp64 peak (the serial pivot and column chains
            # bound it, not HBM)
            R_, C_ = m.W.shape[-2], m.W.shape[-1]
            bs = 128
            upd = sum(2 * R_ * min(bs, C_ - i) * (C_ - min(i + bs, C_)) for i in range(0, C_, bs))
            rooflines[f"solve_and_pack_{m.name}"] = _roofline(
                f"GPTQ solve + pack '{m.name}' (affine: fp64 Cholesky-inverse + column loop + "
                f"fp32 lazy update)", "fp64", 2 * C_ ** 3 / 3 + upd, ms)
            continue
        # bf16 W in; f32 W_dq, u8 code, E8M0 scale and the packed code out
        byt = n * (MXFP_BYTES_PER_ELEMENT + m.pack_bits / 8)
        rooflines[f"solve_and_pack_{m.name}"] = _roofline(
            f"GPTQ solve + pack '{m.name}' ({m.solve['mode']})", "hbm", byt, ms)
    dom = max(rooflines, key=lambda k: rooflines[k]["launch_ms"])
    if dom.startswith("hessian_"):
        # the profile's largest SYRK dispatch is the dominant Hessian
        rooflines[dom]["traffic"] = _traffic(tag, "mgq::syrk_kernel<false")
    cpu = (_cpu_baseline_dense(L, out[:2], out[2], args.cpu_seconds, not args.cpu_sample)
           if args.cpu_seconds > 0 else None)
    config = {"workload": L.name, "elements": elements,
              "matrices": {m.name: list(m.W.shape[1:]) for m in L.mats},
              "tokens": {k: int(X.shape[0]) for k, X in L.inputs.items()}}
    extra = {"phase_rooflines": rooflines}
    # rocprofv3 counters of this config's committed profile (one SYRK
    # dispatch per calibration input, in the step's launch order)
    utils = _counters_in_order(tag, "mgq::syrk_kernel<false", "mfma_util_pct")
    if len(utils) == len(keys):
        extra["hessian_mfma_util_pct"] = dict(zip(keys, utils))
    busy = _counters_in_order(tag, "mgq::mxfp_solve_kernel", "valu_busy_pct")
    busy += _counters_in_order(tag, "mgq::affine_block_kernel", "valu_busy_pct")
    if busy:
        extra["solve_valu_busy_pct"] = max(busy)
    _line(args, value, ms_step, config, phases, rooflines[dom], cpu, setup_s, extra)
    return 0


def _cpu_baseline_dense(L, gpu_out, Hs, budget_s, full=True):
    """CPU oracle on the whole layer (full) or on a bounded sample scaled
    linearly. full: every Hessian whose dense count 2 N C^2 is at most 2e14
    flops on all its tokens, a larger one on its first 65536 tokens (its cost
    is linear in tokens), every solve + pack on all rows. Sampled: each
    Hessian on the first tokens that fit the budget and each solve + pack on
    the first 2048 rows with the full Hessian (the column loops are
    elementwise over rows); the affine path always solves all rows."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import gptq_ref, hessian_ref, packing_ref

    info = _cpu_setup(torch)
    res, _ = gpu_out
    t_total, agree_n, agree_d, parts = 0.0, 0, 0, []
    per_budget = budget_s / (len(L.inputs) + len(L.mats))
    sampled = False
    for k, X in L.inputs.items():
        N, C = X.shape
        if full and 2.0 * N * C * C <= 2e14:
            n_s = N
        elif full:  # a 65536-token sample, scaled linearly in tokens
            n_s = min(N, 65536)
        else:
            n_s = int(min(N, max(256, per_budget * 0.9e12 / (2.0 * C * C))))
        sampled |= n_s < N
        xs = X[:n_s].cpu()
        t = time.perf_counter()
        hessian_ref.stash_hessian([xs], C)
        dt = time.perf_counter() - t
        t_total += dt * N / n_s
        parts.append(f"Hessian '{k}' on {n_s}/{N} tokens")
        print(f"cpu leg: {parts[-1]}: {dt:.1f} s", file=sys.stderr, flush=True)
    for m, r in zip(L.mats, res):
        R, C = m.W.shape[1:]
        kw = dict(m.solve)
        H = Hs[m.inp].cpu()
        r_s = R if (kw["mode"] == "affine" or full) else int(min(R, 2048))
        sampled |= r_s < R
        Ws = m.W[0, :r_s].unsqueeze(0).cpu()
        t = time.perf_counter()
        rq = gptq_ref.solve_gptq(Ws, H.clone(), **kw)[0]
        packing_ref.pack_q(rq[0].numpy(), m.pack_bits)
        dt = time.perf_counter() - t
        t_total += dt * R / r_s
        agree_n += int((r[0][0, :r_s].cpu() == rq[0]).sum())
        agree_d += rq.numel()
        parts.append(f"solve+pack '{m.name}' on {r_s}/{R} rows")
        print(f"cpu leg: {parts[-1]}: {dt:.1f} s", file=sys.stderr, flush=True)
    return {
        "value": round(L.elements / t_total, 1),
        "unit": "elements/s",
        **info,
        "kind": "port",
        "extrapolated": sampled,
        "sample": ("CPU oracle, extrapolated linearly from " if sampled else "CPU oracle, timed in full: ")
                  + "; ".join(parts) + f" ({'estimated ' if sampled else ''}{t_total:.1f} s per layer)",
        "code_agreement_with_gpu": round(agree_n / max(agree_d, 1), 6),
    }


def run_gemm_ceiling(args, torch):
    """bf16 GEMMs through torch (hipBLASLt on ROCm), fp32 accumulation, timed
    with events over args.steps launches after args.warmup: a square
    8192^3 product, the config-4 gate_up Gram matrix of all 1048576 routed
    rows as one [2048 x 1048576] x [1048576 x 2048] product, and 128
    per-expert [2048 x 8192] x [8192 x 2048] products as one bmm (operands
    contiguous). Full products: twice the flops of the lower triangle the
    SYRK computes."""
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(5)
    cases = []
    a = torch.randn(8192, 8192, generator=g, device=dev).to(torch.bfloat16)
    b = torch.randn(8192, 8192, generator=g, device=dev).to(torch.bfloat16)
    cases.append(("square 8192^3", lambda: torch.matmul(a, b), 2 * 8192 ** 3))
    X = torch.randn(1048576, 2048, generator=g, device=dev).to(torch.bfloat16)
    XT = X.t().contiguous()
    cases.append(("gram [2048 x 1048576] x [1048576 x 2048]", lambda: torch.matmul(XT, X),
                  2 * 2048 * 2048 * 1048576))
    Xe = X.view(128, 8192, 2048)
    XeT = Xe.transpose(1, 2).contiguous()
    cases.append(("128 x gram [2048 x 8192] x [8192 x 2048] (bmm)", lambda: torch.bmm(XeT, Xe),
                  2 * 128 * 2048 * 2048 * 8192))
    out = []
    for name, fn, flops in cases:
        for _ in range(max(args.warmup, 1)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        out.append({"case": name, "ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                    "frac_of_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)})
        print(json.dumps(out[-1]), flush=True)
    print(json.dumps({"metric": "bf16 GEMM ceiling (torch.matmul / bmm, hipBLASLt)", "unit": "TFLOP/s",
                      "peak": PEAK_BF16_TFLOPS, "steps": args.steps, "cases": out}))
    return 0


def main(argv=None) -> int:
    args = _args(argv)
    if args.gpus != 1:
        print(f"bench.py measures a single GPU (got --gpus {args.gpus}); multi-GPU runs are out of "
              "scope for this build (experts shard across GPUs with no exchange)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from mlx_gptq import _native

    _native.load()
    torch.cuda.set_device(torch.device("cuda", 0))
    if args.gemm_ceiling:
        return run_gemm_ceiling(args, torch)
    if args.audit:
        if args.config != 4:
            print("--audit measures the config-4 layer only", file=sys.stderr)
            return 2
        return run_audit(args, torch, np)
    if args.capture:
        if args.config != 4:
            print("--capture measures the routed (config 4) layer only", file=sys.stderr)
            return 2
        return run_capture(args, torch, np)
    if args.config == 4:
        return run_moe(args, torch, np)
    return run_dense(args, torch, np)


if __name__ == "__main__":
    sys.exit(main())

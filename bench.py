#!/usr/bin/env python3
"""Benchmark of the VNN propagation step on one MI355X (BASELINE.json metric).

Workload: 62x62 ALU chip, ROI 40x50, K = 23x13, M = 16 Green's filters,
d = 4, B = 128, fp32, continuous Codd mode, output port widened to 8x2 = 16 target cells.
A *step* is one optimiser step of the reference's VNNTrainer.train_step: forward, MSE loss,
reverse pass and the AdamW update, on a batch already resident in HBM.  The whole step is
captured once in a HIP graph and replayed.

Also reported: eval samples/s (config 1: B = 1024, ste_ternary, tau = 0.1, forward only, and
the same at B = 128), per-kernel-family device times with their roofline against 8 TB/s, and
the CPU baseline (the float32 NumPy/scipy.fft restatement in ``oracle/``, timed on this
host's cores).  Prints exactly one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "neurocell-v2_amd"))

METRIC = "train ms/step & eval samples/s at 62x62 ALU B=128; % of HBM roofline"
HBM_PEAK_GBS = 8000.0


def synthetic(name, seed, B=None):
    """Seeded inputs of a BASELINE workload (neurocell.configs): W~N(0,0.1), B~N(0,0.01),
    S~N(0,1) on (3,H,W); filters ~N(0,1/K) (variance 1/K); port inputs and target bits."""
    from neurocell.configs import CONFIGS
    return CONFIGS[name].synthetic(seed, batch=B)


def algorithmic_bytes(B, M, N, F, hb=0, dx=1, P=16):
    """Per-call algorithmic bytes (each interface operand counted once, 4 B/f32, 8 B/c64).
    spectra: the state x in (once, however many partial planes hold it), the border spectrum
    in, xhat out.  conv_epilogue_fwd: xhat and ghat in, w/s/b in, z out (training), the
    step's output x' out (once), mean/rstd out.  conv_port_fwd (the last step): xhat, ghat,
    port indices and parameters in, z out (training), zo, mean/rstd and the outputs out.
    fftconv_bwd: gz, xhat, ghat in, dx out, dghat read-modify-write, the cotangent spectrum
    sum out.  The step's epilogues run without a border term (hb = 0: it is folded into the
    spectra)."""
    return {
        "spectra": 4 * B * N + 8 * F + 8 * B * F,
        "conv_epilogue_fwd": 8 * B * F + 8 * M * F + 12 * N + 4 * B * M * N + 4 * B * N
                             + 8 * B * M,
        "conv_port_fwd": 8 * B * F + 8 * M * F + 4 * B * M * N + 16 * P + 4 * B * M * P
                         + 8 * B * M + 4 * B * P,
        "fftconv_bwd": (4 * B * M * N + 8 * B * F + 8 * M * F + dx * 4 * B * N + 16 * M * F
                        + 8 * M * F),
        "epilogue_fwd": 4 * (B * M * N + hb * M * N + 3 * N + B * N + 2 * B * M),
        "epilogue_bwd": 4 * (2 * B * M * N + hb * M * N + 6 * N + 2 * B * M + B * N),
        "port_fwd": 4 * (B * M * N + hb * M * N + 2 * B * M + B * M * P),
        "port_bwd": 4 * (2 * B * M * N + hb * M * N + 4 * B * M + B * M * P),
    }


def time_family(fn, reps, torch):
    """Average device time of fn() over reps back-to-back launches on the current stream."""
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e3  # us


def kernel_families(ts, torch, reps):
    """Device time per call of each C-ABI family at the step's shapes (after a step, so every
    operand holds real data)."""
    from neurocell._lib import call, ptr, stream_ptr
    p = ts.plan
    B, M, h, w = p.B, p.M, p.h, p.w
    fh, fw = p.fft
    t = 1
    s = stream_ptr
    ws_ep, n_ep = ptr(p.ws_epi), p.ws_epi.numel() * 4
    ws_fc, n_fc = ptr(p.ws_fc), p.ws_fc.numel() * 4
    fams = {
        "spectra": lambda: call("nc_fftconv_spectra", s(), B, h, w, fh, fw, ptr(p.xs[t]), p.G,
                                ptr(p.border_hat), ptr(p.xhat[t])),
        "conv_epilogue_fwd": lambda: call("nc_fftconv_epilogue_fwd", s(), B, M, h, w, p.cp[0],
                                          p.cp[1], fh, fw, ptr(p.xhat[t]), ptr(p.ghat), p.act,
                                          p.slope, ptr(p.w_eff), ptr(p.s_eff), ptr(p.b_roi),
                                          ptr(p.zs[t]), ptr(p.xs[t + 1]), ptr(p.mean[t]),
                                          ptr(p.rstd[t]), ws_ep, n_ep),
        "conv_port_fwd": lambda: call("nc_fftconv_port_fwd", s(), B, M, h, w, p.cp[0], p.cp[1],
                                      fh, fw, ptr(p.xhat[t]), ptr(p.ghat), p.fact, p.fslope, p.P,
                                      ptr(p.port_idx), ptr(p.pp), ptr(p.zs[-1]), ptr(p.out),
                                      ptr(p.zo), ptr(p.mean[-1]), ptr(p.rstd[-1]), ptr(p.pre),
                                      ws_ep, n_ep),
        "fftconv_bwd": lambda: call("nc_fftconv_bwd_parts", s(), B, M, h, w, h, w, p.cp[0],
                                    p.cp[1], fh, fw, ptr(p.gz), ptr(p.xhat[t]), ptr(p.ghat), 1,
                                    ptr(p.gy[0]), ptr(p.rows["dg"]), 0, 0, ptr(p.rows["gd"]),
                                    0, ws_fc, n_fc),
        "epilogue_bwd": lambda: call("nc_epilogue_bwd_parts", s(), B, M, h, w, p.act, p.slope,
                                     0, ptr(p.zs[t]), None, ptr(p.w_eff), ptr(p.s_eff),
                                     ptr(p.b_roi), ptr(p.mean[t]), ptr(p.rstd[t]),
                                     ptr(p.gy[1]), ptr(p.gz), ptr(p.pg_rows),
                                     p.pg_rows[0].numel(), ws_ep, n_ep),
        "port_bwd": lambda: call("nc_port_bwd_parts", s(), B, M, h, w, 0, p.fact, p.fslope,
                                 p.P, ptr(p.port_idx), ptr(p.zs[-1]), None, ptr(p.pp),
                                 ptr(p.zo), ptr(p.mean[-1]), ptr(p.rstd[-1]), ptr(p.pre),
                                 ptr(p.g_out), ptr(p.gz), ptr(p.pp_rows), B * p.P, ws_ep,
                                 n_ep),
    }
    per_step = {"spectra": p.d - 1, "conv_epilogue_fwd": p.d - 1, "conv_port_fwd": 1,
                "fftconv_bwd": p.d, "epilogue_bwd": p.d - 1, "port_bwd": 1}
    return {k: (time_family(f, reps, torch), per_step[k]) for k, f in fams.items()}


# C-ABI family of each kernel of a --families-only run (k_batch_reduce belongs to whichever
# backward family launched it: the preceding kernel decides).
_FAMILY_KERNELS = {
    "spectra": ("k_wrfft2", "k_lrfft2", "k_prfft2"),
    "conv_epilogue_fwd": ("k_pconv_epi", "k_epi_fwd", "k_group_sum", "k_tile_stats",
                          "k_tile_fwd"),
    "conv_port_fwd": ("k_pconv_port", "k_wconv_fwd", "k_linv_conv", "k_pconv_fwd",
                      "k_port_fwd", "k_port_combine", "k_port_fwd_tiled"),
    "fftconv_bwd": ("k_wbwd_part", "k_psum", "k_wbwd_dx_fin", "k_wbwd_dg_red", "k_wbwd_dg_sum",
                    "k_lred", "k_linv_dx", "k_pspec", "k_pbwd_red", "k_pdx_half"),
    "epilogue_bwd": ("k_epi_bwd", "k_tile_bwd1", "k_tile_bwd2"),
    "port_bwd": ("k_port_bwd",),
}


def traffic_summary(fetch_dir, write_dir, reps, out_path):
    """HBM bytes per launch of each kernel family from two rocprofv3 counter passes (FETCH_SIZE,
    WRITE_SIZE, KiB per dispatch) over `bench.py --families-only --kernel-reps reps`, scaled by
    what the counters read for the run's 256 MiB device copies.  Writes out_path (JSON)."""
    import csv

    def load(d, counter):
        rows = list(csv.DictReader(open(os.path.join(d, "run_counter_collection.csv"))))
        per = {}
        for r in rows:
            if r["Counter_Name"] != counter:
                continue
            key = int(r["Dispatch_Id"])
            name = r["Kernel_Name"].replace("(anonymous namespace)::", "").replace("void ", "")
            per[key] = (name, per.get(key, ("", 0.0))[1] + float(r["Counter_Value"]))
        return [per[k] for k in sorted(per)]

    res = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        seq = load(d, counter)
        copies = [v for n, v in seq if "copyBuffer" in n and v > 1e5]
        scale = (64 << 20) * 4 / (float(np.median(copies)) * 1024.0)
        fam_kib, last = {}, None
        start = max(i for i, (n, _) in enumerate(seq) if "copyBuffer" in n) + 1
        for name, kib in seq[start:]:
            fam = next((f for f, ks in _FAMILY_KERNELS.items()
                        if any(name.startswith(k) for k in ks)), None)
            if name.startswith("k_batch_reduce"):
                fam = last
            if fam is None:
                continue
            last = fam
            fam_kib[fam] = fam_kib.get(fam, 0.0) + kib
        res[counter] = {f: v * 1024.0 * scale / (reps + 1) for f, v in fam_kib.items()}
        res[counter + "_scale"] = scale
    ab = algorithmic_bytes(128, 16, 2000, 64 * 33, P=16)
    out = {"_calibration": {"copy_bytes": (64 << 20) * 4, "fetch_scale": round(res["FETCH_SIZE_scale"], 4),
                            "write_scale": round(res["WRITE_SIZE_scale"], 4),
                            "calls_per_family": reps + 1}}
    for f in _FAMILY_KERNELS:
        fb, wb = res["FETCH_SIZE"].get(f, 0.0), res["WRITE_SIZE"].get(f, 0.0)
        out[f] = {"fetch_bytes": int(fb), "write_bytes": int(wb), "traffic_bytes": int(fb + wb),
                  "algorithmic_bytes": ab[f],
                  "traffic_over_algorithmic": round((fb + wb) / ab[f], 2)}
    with open(out_path, "w") as fh:
        json.dump(out, fh, indent=1)
    return out


def cpu_baseline(seed, B, budget_s):
    """Float32 NumPy + scipy.fft restatement (oracle/) of one config-0 train step on this
    host's cores: forward, MSE loss, reverse pass and AdamW.  Timed over a bounded sample."""
    from oracle import vnn_oracle as O
    cores = len(os.sched_getaffinity(0))
    cell, filt, x, y = synthetic("config0", seed, B)
    geom = O.alu_geometry(out_width=2)
    m = np.zeros(cell.size + filt.size, np.float32)
    v = np.zeros_like(m)
    theta = np.concatenate([cell.ravel(), filt.ravel()])
    times = []
    with O.precision(np.float32, workers=cores):
        t_end = time.perf_counter() + budget_s
        count = 0
        while True:
            t0 = time.perf_counter()
            c = theta[:cell.size].reshape(cell.shape)
            f = theta[cell.size:].reshape(filt.shape)
            fwd = O.propagate(c, f, x, geom)
            _, g_out = O.mse_loss(fwd[0], y)
            _, gc, gf = O.propagate_vjp(c, f, x, geom, g_out.astype(np.float32), fwd=fwd)
            g = np.concatenate([gc.ravel(), gf.ravel()]).astype(np.float32)
            theta, m, v, count = O.adamw_step(theta, g, m, v, count, 1e-3)
            theta = theta.astype(np.float32)
            times.append(time.perf_counter() - t0)
            if time.perf_counter() > t_end and len(times) >= 2:
                break
    return {"value": round(1e3 * float(np.median(times)), 3), "unit": "ms/step", "cores": cores,
            "kind": "port",
            "sample": f"{len(times)} config-0 train steps (B={B}, fwd+bwd+AdamW), float32 "
                      f"NumPy + scipy.fft restatement in oracle/, scipy.fft workers={cores}, "
                      "median reported"}


def run_config(name, args, torch):
    """Times one BASELINE workload at its full size (neurocell.configs): a HIP-graph-replayed
    train step (or, for config 1, a forward evaluation batch) and each C-ABI kernel family at
    the step's shapes.  Prints one JSON line; not the headline figure."""
    from neurocell.configs import CONFIGS
    from neurocell.engine import (EvalState, ParamState, StepPlan, TrainState, flatten_inputs,
                                  port_input_shapes)
    cfg = CONFIGS[name]
    dev = torch.device("cuda")
    topo = cfg.topology()
    cell, filt, x, y = cfg.synthetic(0)
    xt = torch.from_numpy(x).to(dev)
    B = x.shape[0]
    plan = StepPlan(topo, B, port_input_shapes(xt, topo), roi_bbox=cfg.roi_bbox,
                    training=cfg.train)
    ps = ParamState(torch.from_numpy(cell).to(dev), torch.from_numpy(filt).to(dev),
                    learning_rate=1e-3)
    if cfg.train:
        st = TrainState(plan, ps, codd_mode=cfg.codd_mode, state_temperature=cfg.tau)
        st.y.copy_(torch.from_numpy(y.reshape(B, -1)).to(dev))
        run = st.step
    else:
        st = EvalState(plan, ps.cell, ps.filt, codd_mode=cfg.codd_mode,
                       state_temperature=cfg.tau)
        run = st.run
    st.x.copy_(flatten_inputs(xt, topo))
    if not args.no_graph:
        st.capture()
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        run()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    rec = {"config": name, "batch": B, "grid": list(topo.grid_shape), "roi": [plan.h, plan.w],
           "kernel": list(cfg.kernel), "directions": plan.M, "depth": plan.d,
           "fft": list(plan.fft), "codd_mode": cfg.codd_mode, "train": cfg.train,
           "steps": args.steps, "ms_per_step": round(wall_ms, 4),
           "device_ms_per_step": round(e0.elapsed_time(e1) / args.steps, 4),
           "samples_per_s": round(B / wall_ms * 1e3, 1)}
    if cfg.train:
        loss = float(plan.loss.item())
        if not np.isfinite(loss):
            raise RuntimeError(f"non-finite loss {loss}")
        rec["final_loss"] = round(loss, 6)
        fams = kernel_families(st, torch, args.kernel_reps)
        ab = algorithmic_bytes(B, plan.M, plan.N, plan.F, P=plan.P)
        rec["kernels"] = {k: {"us_per_call": round(us, 2), "calls_per_step": n,
                              "algorithmic_MB": round(ab[k] / 1e6, 3),
                              "GBps": round(ab[k] / (us * 1e-6) / 1e9, 1),
                              "frac_hbm": round(ab[k] / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
                          for k, (us, n) in fams.items()}
    print(json.dumps(rec))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-baseline leg")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly, no HIP graph")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline")
    ap.add_argument("--kernel-reps", type=int, default=200)
    ap.add_argument("--no-eval", action="store_true", help="skip the evaluation legs")
    ap.add_argument("--config", default=None,
                    help="time one BASELINE workload of neurocell.configs at full size "
                         "(config0..config4, config2_literal) instead of the headline line")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"), default=None,
                    help="summarise two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) of a "
                         "--families-only run into profiles/traffic_config0.json and exit")
    ap.add_argument("--families-only", action="store_true",
                    help="profiling aid: one eager train step, a 256 MiB device copy (the "
                         "traffic-counter calibration), then --kernel-reps calls of each "
                         "kernel family; prints a one-line note, no JSON")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU (--gpus {args.gpus} requested); "
              "the data-parallel sharding over B is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)

    if args.traffic:
        out = traffic_summary(args.traffic[0], args.traffic[1], args.kernel_reps,
                              os.path.join(ROOT, "profiles", "traffic_config0.json"))
        print(json.dumps({k: v.get("traffic_over_algorithmic") for k, v in out.items()
                          if k != "_calibration"}))
        return
    import torch
    if args.config:
        run_config(args.config, args, torch)
        return
    from neurocell.engine import (EvalState, ParamState, StepPlan, TrainState, flatten_inputs,
                                  port_input_shapes)
    from neurocell.topology import ChipTopology2D

    dev = torch.device("cuda")
    topo = ChipTopology2D.alu_chip(n=8, kernel_size=(23, 13), directions=16, depth=4,
                                   out_width=2)
    B = 128
    cell, filt, x, y = synthetic("config0", 0, B)
    xt = torch.from_numpy(x).to(dev)
    plan = StepPlan(topo, B, port_input_shapes(xt, topo), training=True)
    ps = ParamState(torch.from_numpy(cell).to(dev), torch.from_numpy(filt).to(dev),
                    learning_rate=1e-3)
    ts = TrainState(plan, ps)
    ts.x.copy_(flatten_inputs(xt, topo))
    ts.y.copy_(torch.from_numpy(y.reshape(B, -1)).to(dev))
    if args.families_only:
        ts.step()
        src = torch.empty(64 << 20, device=dev, dtype=torch.float32).normal_()
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        fams = kernel_families(ts, torch, args.kernel_reps)
        torch.cuda.synchronize()
        print("families-only: copy 256 MiB x3; " + ", ".join(
            f"{k} {us:.1f} us" for k, (us, _) in fams.items()))
        return
    if not args.no_graph:
        ts.capture()
    for _ in range(args.warmup):
        ts.step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        ts.step()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    dev_ms = e0.elapsed_time(e1) / args.steps
    loss = float(ts.plan.loss.item())
    if not np.isfinite(loss):
        raise RuntimeError(f"non-finite loss {loss}")

    # evaluation throughput (config 1 and config 0 batch)
    evals = {}
    eval_cases = () if args.no_eval else (
        ("config1_B1024_ste_ternary", 1024, "ste_ternary", 0.1),
        ("B128_continuous", 128, "continuous", 1.0))
    for name, eb, mode, tau in eval_cases:
        _, _, xe, _ = synthetic("config1", 1, eb)
        xet = torch.from_numpy(xe).to(dev)
        ep = StepPlan(topo, eb, port_input_shapes(xet, topo), training=False)
        es = EvalState(ep, ps.cell, ps.filt, codd_mode=mode, state_temperature=tau)
        es.x.copy_(flatten_inputs(xet, topo))
        if not args.no_graph:
            es.capture()
        reps = max(20, args.steps // 2)
        for _ in range(5):
            es.run()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            es.run()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / reps
        evals[name] = {"ms_per_batch": round(ms, 4), "samples_per_s": round(eb / ms * 1e3, 1)}

    # per-family device times and the roofline of the dominant one
    fams = kernel_families(ts, torch, args.kernel_reps)
    F = plan.F
    ab = algorithmic_bytes(B, plan.M, plan.N, F, P=plan.P)
    share = {k: us * n for k, (us, n) in fams.items()}
    dom = max(share, key=share.get)
    us = fams[dom][0]
    achieved = ab[dom] / (us * 1e-6) / 1e9
    kernels = {k: {"us_per_call": round(us_, 2), "calls_per_step": n,
                   "algorithmic_MB": round(ab[k] / 1e6, 3),
                   "GBps": round(ab[k] / (us_ * 1e-6) / 1e9, 1),
                   "frac_hbm": round(ab[k] / (us_ * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
               for k, (us_, n) in fams.items()}
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_config0.json")
    if os.path.exists(tpath):
        with open(tpath) as fh:
            entry = json.load(fh).get(dom)
        # HBM bytes per launch from the FETCH_SIZE / WRITE_SIZE counter passes, scaled by
        # what the counters read for a plain 256 MiB copy
        traffic = entry.get("traffic_bytes") if isinstance(entry, dict) else None

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(0, B, args.cpu_budget)

    rec = {
        "metric": METRIC,
        "value": round(wall_ms, 4),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded BASELINE config-0 distributions; resident in HBM)",
        "config": {"workload": "config0: 62x62 ALU, ROI 40x50, K=23x13, M=16, d=4, B=128, "
                               "fp32, continuous Codd, 16-cell output port; train step = "
                               "fwd + MSE + bwd + AdamW, HIP-graph replay",
                   "global_batch": B, "grid": [62, 62], "roi": [40, 50], "kernel": [23, 13],
                   "directions": 16, "depth": 4, "fft": list(plan.fft),
                   "graph": not args.no_graph},
        "device_ms_per_step": round(dev_ms, 4),
        "final_loss": round(loss, 6),
        "eval": evals,
        "eval_samples_per_s": (evals["config1_B1024_ste_ternary"]["samples_per_s"]
                               if evals else None),
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec))


if __name__ == "__main__":
    main()

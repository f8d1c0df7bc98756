"""Whole-step parity at the benchmark batch sizes on the MI355X: the exact workloads that
``bench.py`` times (configs 0, 1 and 4 at their full batch, config 3 at its full 32
directions, config 2 at its full 16), through the C ABI, against the float64 oracle.

Batch-dependent code paths are the point: at B >= 512 the single-pass epilogue kernels run
one workgroup per sample with every direction in registers (the config-4 train step and the
config-1 evaluation), below it the directions split over several workgroups; the reduction
trees over samples change shape with B as well.

The oracle runs over sample chunks on a thread pool (``helpers.oracle_*_batched``): samples
are independent in the forward pass and the parameter gradients are sums over samples, so
the chunked oracle equals one call on the whole batch.

Bars: forward states rel-L2 <= 1e-5 (every step state x_t, t >= 1,
and the port outputs), parameter gradients rel-L2 <= 1e-4.  One exception, measured and
stated: config 3's 16 port outputs after 8 steps on 256x256 grids carry more rounding than
1e-5 in any fp32 evaluation - the oracle's own algorithm run in float32 (NumPy + pocketfft)
lands at 1.6e-5 there - so its port outputs are held to the larger of 1e-5 and 1.25x that
float32 restatement's error, measured in the test; its states still meet 1e-5.
"""
import numpy as np
import pytest
import torch

from helpers import config_geometry, oracle_forward_batched, oracle_vjp_batched, rel_l2

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-5
GRAD_TOL = 1e-4


def _fp32_restatement_error(cell, filt, x, geom, **kw):
    """rel-L2 of the oracle's algorithm evaluated in float32 against float64: the rounding any
    fp32 implementation of the same maths carries."""
    from oracle import vnn_oracle as O
    ref = O.propagate(cell, filt, x, geom, **kw)[0]
    with O.precision(np.float32, workers=8):
        f32 = O.propagate(cell, filt, x, geom, **kw)[0]
    return rel_l2(f32, ref)


def _train_step(name, seed, batch=None, directions=None, out_tol=FWD_TOL):
    from neurocell.configs import CONFIGS
    from neurocell.engine import StepPlan, flatten_inputs, inv_tau_f32, port_input_shapes
    cfg = CONFIGS[name]
    cell, filt, x, _ = cfg.synthetic(seed, batch=batch, directions=directions)
    B = x.shape[0]
    topo = cfg.topology(directions=directions)
    geom = config_geometry(cfg, directions=directions)
    g_out = np.random.default_rng(seed + 100).normal(size=(B,) + geom.out_size)
    g_out = g_out.astype(np.float32)
    print(f"[{name}] B={B} M={filt.shape[0]} bbox={cfg.roi_bbox} mode={cfg.codd_mode}",
          flush=True)
    dev = torch.device("cuda")
    xt = torch.from_numpy(x).to(dev)
    plan = StepPlan(topo, B, port_input_shapes(xt, topo), roi_bbox=cfg.roi_bbox,
                    training=True)
    c, f = torch.from_numpy(cell).to(dev), torch.from_numpy(filt).to(dev)
    it = inv_tau_f32(cfg.tau)
    out = plan.forward(c, f, flatten_inputs(xt, topo), codd_mode=cfg.codd_mode, inv_tau=it)
    gc, gf = torch.empty_like(c), torch.empty_like(f)
    plan.backward(c, f, torch.from_numpy(g_out.reshape(B, -1)).to(dev), gc, gf,
                  codd_mode=cfg.codd_mode, inv_tau=it)
    torch.cuda.synchronize()
    # the step states t >= 1: the sum of the hidden epilogue's direction-group partials
    states = [plan.xs[t].sum(0).cpu().numpy() for t in range(1, plan.d)]
    out, gc, gf = out.cpu().numpy(), gc.cpu().numpy(), gf.cpu().numpy()
    kw = dict(roi_bbox=cfg.roi_bbox, mode=cfg.codd_mode, tau=cfg.tau)
    r_out, r_gc, r_gf = oracle_vjp_batched(cell, filt, x, geom, g_out, **kw)
    _, r_xs = oracle_forward_batched(cell, filt, x, geom, states=True, **kw)
    errs = {"out": rel_l2(out, r_out.reshape(B, -1)), "gW": rel_l2(gc[0], r_gc[0]),
            "gB": rel_l2(gc[1], r_gc[1]), "gS": rel_l2(gc[2], r_gc[2]), "gG": rel_l2(gf, r_gf)}
    errs.update({f"x{t}": rel_l2(states[t - 1], r_xs[t]) for t in range(1, plan.d)})
    print(f"[{name}] {errs}", flush=True)
    assert errs["out"] < out_tol, errs
    for t in range(1, plan.d):
        assert errs[f"x{t}"] < FWD_TOL, errs
    for k in ("gW", "gB", "gS", "gG"):
        assert errs[k] < GRAD_TOL, errs
    return plan


def test_config4_train_step_b512():
    """Config 4 exactly as benchmarked: B = 512, the 24x32 crop (6, 30, 10, 42), ste_binary at
    tau = 0.1.  The hidden epilogue's backward takes the one-workgroup-per-sample branch."""
    from neurocell._lib import lib
    assert lib().nc_epilogue_bwd_partials(512, 16, 24, 32) == 512  # one group per sample
    assert lib().nc_epilogue_bwd_partials(128, 16, 24, 32) > 128   # the split branch
    _train_step("config4", 4)


def test_config0_train_step_b128():
    """Config 0 exactly as benchmarked: B = 128, the full 40x50 ROI, continuous."""
    _train_step("config0", 0)


def test_config3_step_m32():
    """Config 3's 32 directions (tiled Chan epilogue over 49 tiles of 1024 cells, two-segment
    256x256 transforms, three 16-direction reduction chunks) at a small batch.  The port
    outputs are held to the rounding of an fp32 restatement (module docstring)."""
    from neurocell.configs import CONFIGS
    cfg = CONFIGS["config3"]
    cell, filt, x, _ = cfg.synthetic(3, batch=2)
    e32 = _fp32_restatement_error(cell, filt, x, config_geometry(cfg), roi_bbox=cfg.roi_bbox,
                                  mode=cfg.codd_mode, tau=cfg.tau)
    print(f"[config3] fp32 restatement port rel-L2 {e32:.3e}", flush=True)
    _train_step("config3", 3, batch=2, out_tol=max(FWD_TOL, 1.25 * e32))


def test_config2_step_m16():
    """Config 2's 16 directions (K = 63x63, 112x112 ROI, 256x256 grid, d = 8) at a small
    batch."""
    _train_step("config2", 2, batch=4)


def test_config1_eval_b1024():
    """Config 1 exactly as benchmarked: the evaluation plan (training=False: z never reaches
    HBM, the correlation and the epilogue fused) at B = 1024, ste_ternary at tau = 0.1,
    compared by rel-L2 on the port outputs."""
    from neurocell.configs import CONFIGS
    from neurocell.engine import EvalState, StepPlan, flatten_inputs, port_input_shapes
    cfg = CONFIGS["config1"]
    cell, filt, x, _ = cfg.synthetic(1)
    B = x.shape[0]
    assert B == 1024
    topo = cfg.topology()
    dev = torch.device("cuda")
    xt = torch.from_numpy(x).to(dev)
    plan = StepPlan(topo, B, port_input_shapes(xt, topo), training=False)
    c, f = torch.from_numpy(cell).to(dev), torch.from_numpy(filt).to(dev)
    ev = EvalState(plan, c, f, cfg.codd_mode, cfg.tau)
    ev.x.copy_(flatten_inputs(xt, topo))
    out = ev.run().cpu().numpy()
    states = [plan.xs[t].sum(0).cpu().numpy() for t in range(1, plan.d)]
    ev.capture()  # the benchmarked form: a replayed HIP graph
    rep = []
    for _ in range(3):
        rep.append(ev.run().cpu().numpy())
        torch.cuda.synchronize()
    ref, r_xs = oracle_forward_batched(cell, filt, x, config_geometry(cfg), states=True,
                                       mode=cfg.codd_mode, tau=cfg.tau)
    errs = {"out": rel_l2(out, ref.reshape(B, -1))}
    errs.update({f"x{t}": rel_l2(states[t - 1], r_xs[t]) for t in range(1, plan.d)})
    print(f"[config1] B={B} {errs}", flush=True)
    for k, v in errs.items():
        assert v < FWD_TOL, errs
    for r in rep:
        assert np.array_equal(r, out)

"""Python API parity on the MI355X: the reference-named operators, propagation, model and
trainer (all running the HIP kernels through the C ABI) against the float64 oracle, plus
graph-replay checks of the trainer against its own eager launches.

Bars: forward rel-L2 <= 1e-5, gradients rel-L2 <= 1e-4; optimiser
trajectories (AdamW normalises each update, so tiny gradients are amplified) <= 1e-3 on the
parameter change; graph replays bit-identical to eager launches.
"""
import types

import numpy as np
import pytest
import torch

from helpers import alu_case, rel_l2
from oracle import vnn_oracle as O

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-5
GRAD_TOL = 1e-4
TRAJ_TOL = 1e-3
CROP = (6, 30, 10, 42)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def mask(bbox):
    return None if bbox is None else types.SimpleNamespace(roi_bbox=bbox, is_full_roi=False)


# ------------------------------------------------------------------ operators

@pytest.mark.parametrize("act,hb", [("tanh", True), ("gelu", False), ("leaky_relu", True)])
def test_roi_epilogue_autograd(act, hb):
    from neurocell import pallas_fused_roi_step_epilogue
    rng = np.random.default_rng(1)
    B, M, h, w = 3, 4, 20, 24
    z = rng.normal(size=(B, M, h, w)).astype(np.float32)
    d = rng.normal(size=(1, M, h, w)).astype(np.float32)
    ws, ss, bs = (rng.normal(size=(h, w)).astype(np.float32) for _ in range(3))
    gy = rng.normal(size=(B, h, w)).astype(np.float32)
    ts = [dev(a).requires_grad_() for a in (z, d, ws, ss, bs)]
    out = pallas_fused_roi_step_epilogue(*ts, activate=act, has_border=hb)
    out.backward(dev(gy))
    r_out, mean, rstd = O.epilogue_fwd(z, d, ws, ss, bs, act, hb)
    r = O.epilogue_bwd(z, d, ws, ss, bs, mean, rstd, gy, act, hb)
    assert rel_l2(host(out), r_out) < FWD_TOL
    for t, ref in zip(ts, (r[0], r[1][None], r[2], r[3], r[4])):
        if not hb and t is ts[1]:
            continue
        assert rel_l2(host(t.grad), ref) < GRAD_TOL


@pytest.mark.parametrize("coord", [False, True])
def test_standardize_output_port(coord):
    from neurocell import pallas_standardize_output_port
    rng = np.random.default_rng(2)
    B, M, h, w = 3, 5, 16, 20
    z = rng.normal(size=(B, M, h, w)).astype(np.float32)
    d = rng.normal(size=(1, M, h, w)).astype(np.float32)
    if coord:
        rows, cols = (1, 5, 5, 9, 15), (2, 7, 7, 0, 19)  # a repeated cell adds up
        off, size = (rows, cols), (5, 1)
    else:
        off, size = (4, 11), (3, 2)
        rr, cc = np.meshgrid(np.arange(3) + 4, np.arange(2) + 11, indexing="ij")
        rows, cols = tuple(rr.ravel()), tuple(cc.ravel())
    zt, dt = dev(z).requires_grad_(), dev(d).requires_grad_()
    zo = pallas_standardize_output_port(zt, dt, off, size, True)
    g = rng.normal(size=tuple(zo.shape)).astype(np.float32)
    zo.backward(dev(g))
    # float64 autograd restatement of standardize(z + delta) sampled at the port cells
    z64 = torch.from_numpy(z).double().requires_grad_()
    d64 = torch.from_numpy(d).double().requires_grad_()
    tot = z64 + d64
    mu = tot.mean(dim=(-2, -1), keepdim=True)
    var = ((tot - mu) ** 2).mean(dim=(-2, -1), keepdim=True)
    ref = ((tot - mu) / torch.sqrt(var + 1e-5))[:, :, list(rows), list(cols)]
    ref = ref.reshape(B, M, *size)
    ref.backward(torch.from_numpy(g).double())
    assert rel_l2(host(zo), ref.detach().numpy()) < FWD_TOL
    assert rel_l2(host(zt.grad), z64.grad.numpy()) < GRAD_TOL
    assert rel_l2(host(dt.grad), d64.grad.numpy()) < GRAD_TOL


def _conv_case(seed=3, B=2, M=3, h=20, w=24, kh=7, kw=5):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(B, h, w)).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    gz = rng.normal(size=(B, M, h, w)).astype(np.float32)
    pad = ((kh - 1) // 2, (kw - 1) // 2)
    return x, g, gz, pad


def _check_conv(fn):
    x, g, gz, pad = _conv_case()
    xt, gt = dev(x).requires_grad_(), dev(g).requires_grad_()
    z = fn(xt, gt, pad)
    z.backward(dev(gz))
    with O.precision(np.float64):
        r_z = O.conv2d_direct(x, g[:, 0], pad)
        r_dx, r_dg = O.conv2d_bwd_direct(gz, x, g[:, 0], pad)
    assert rel_l2(host(z), r_z) < FWD_TOL
    assert rel_l2(host(xt.grad), r_dx) < GRAD_TOL
    assert rel_l2(host(gt.grad)[:, 0], r_dg) < GRAD_TOL


def test_pruned_rfft_chain():
    from neurocell import conv2d_pruned_rfft_roi_step, hoist_filter_rfft2_nopad
    fs = (32, 32)

    def fn(x, g, pad):
        kf = hoist_filter_rfft2_nopad(g, g.shape[-2:], pad, fs)
        return conv2d_pruned_rfft_roi_step(x, kf, x.shape[-2:], pad, fs, True)
    _check_conv(fn)


def test_hybrid_nopad_chain():
    from neurocell import conv2d_hybrid_nopad_roi_step, hoist_filter_rfft2_zero_nopad
    fs = (32, 32)

    def fn(x, g, pad):
        token = hoist_filter_rfft2_zero_nopad(g, g.shape[-2:], pad, fs)
        return conv2d_hybrid_nopad_roi_step(x, g.detach(), token, pad, fs, True)
    _check_conv(fn)


def test_small_kernel_step():
    from neurocell import conv2d_small_kernel_roi_step
    _check_conv(lambda x, g, pad: conv2d_small_kernel_roi_step(x, g, pad, True))


@pytest.mark.parametrize("padding", ["VALID", "SAME"])
def test_batched_nchw(padding):
    from neurocell import conv2d_batched_nchw
    x, g, _, pad = _conv_case(seed=4)
    z = conv2d_batched_nchw(dev(x[:, None]), dev(g), padding=padding)
    with O.precision(np.float64):
        if padding == "SAME":
            ref = O.conv2d_direct(x, g[:, 0], pad)
        else:
            ref = O.conv2d_direct(x, g[:, 0], (0, 0))
    assert rel_l2(host(z), ref) < FWD_TOL


def test_need_dx_false_gives_exact_zero_dx():
    """unit_kernels_greens.py:151-156: with need_dx=False the cell cotangent is identically
    zero while the filter gradient still matches the direct correlation's."""
    from neurocell import conv2d_pruned_rfft_roi_step, hoist_filter_rfft2_nopad
    x, g, gz, pad = _conv_case(seed=6)
    fs = (32, 32)
    res = {}
    for need in (True, False):
        xt, gt = dev(x).requires_grad_(), dev(g).requires_grad_()
        kf = hoist_filter_rfft2_nopad(gt, g.shape[-2:], pad, fs)
        z = conv2d_pruned_rfft_roi_step(xt, kf, x.shape[-2:], pad, fs, need)
        z.backward(dev(gz))
        res[need] = (host(xt.grad), host(gt.grad))
    with O.precision(np.float64):
        r_dx, r_dg = O.conv2d_bwd_direct(gz, x, g[:, 0], pad)
    assert float(np.abs(res[False][0]).max()) == 0.0
    assert rel_l2(res[True][0], r_dx) < GRAD_TOL
    assert rel_l2(res[False][1][:, 0], r_dg) < 1e-5
    assert rel_l2(res[False][1], res[True][1]) < 1e-6


def test_no_border_gives_exact_zero_gdb():
    """unit_milestone6_general_vnn.py:107-110: without the border term (has_border=False)
    the border cotangent is identically zero, for the hidden epilogue and the port."""
    from neurocell import pallas_fused_roi_step_epilogue, pallas_standardize_output_port
    rng = np.random.default_rng(8)
    B, M, h, w = 3, 4, 16, 20
    z = rng.normal(size=(B, M, h, w)).astype(np.float32)
    d = rng.normal(size=(1, M, h, w)).astype(np.float32)
    ws, ss, bs = (rng.normal(size=(h, w)).astype(np.float32) for _ in range(3))
    ts = [dev(a).requires_grad_() for a in (z, d, ws, ss, bs)]
    out = pallas_fused_roi_step_epilogue(*ts, activate="tanh", has_border=False)
    out.backward(dev(rng.normal(size=(B, h, w)).astype(np.float32)))
    assert float(ts[1].grad.abs().max()) == 0.0
    assert float(ts[0].grad.abs().max()) > 0.0
    zt, dt = dev(z).requires_grad_(), dev(d).requires_grad_()
    zo = pallas_standardize_output_port(zt, dt, (3, 5), (4, 2), False)
    zo.backward(dev(rng.normal(size=tuple(zo.shape)).astype(np.float32)))
    assert float(dt.grad.abs().max()) == 0.0
    assert float(zt.grad.abs().max()) > 0.0


def test_ste_ternary_zero_thresholding_gap():
    """unit_milestone8_pallas_and_codd.py:240-252 on the device: replacing the raw Codd states
    by discrete values in each ternary regime (1.0 active, 0.3 passive, -1.0 inactive, from
    ``threshold_states``) leaves the ste_ternary forward exactly unchanged."""
    from neurocell import VNNParams, VonNeumannNetwork
    from neurocell.topology import ChipTopology2D
    geom, cell, filt, x, _ = alu_case(21, B=8)
    rng = np.random.default_rng(22)
    cell[2] = rng.uniform(-1.5, 1.5, size=cell[2].shape).astype(np.float32)
    model = VonNeumannNetwork(ChipTopology2D.alu_chip(out_width=2))
    p = VNNParams(dev(cell), dev(filt))
    out_t = model.apply(p, dev(x), codd_mode="ste_ternary", state_temperature=0.25)
    roles = VonNeumannNetwork.threshold_states(p.cell_params[2], active_threshold=0.6)
    one = torch.ones_like(roles)
    s_disc = torch.where(roles >= 2.0, one, torch.where(roles > 0.0, 0.3 * one, -one))
    assert set(np.unique(host(s_disc)).tolist()) == {-1.0, np.float32(0.3), 1.0}
    cell_d = p.cell_params.clone()
    cell_d[2] = s_disc
    out_d = model.apply(VNNParams(cell_d, p.greens_filters), dev(x), codd_mode="ste_ternary",
                        state_temperature=0.25)
    assert float((out_t - out_d).abs().max()) == 0.0
    r_out = O.propagate(cell, filt, x, geom, mode="ste_ternary", tau=0.25)[0]
    assert rel_l2(host(out_t), r_out) < FWD_TOL


def test_circular_ignores_adaptive_crop():
    """propagator.py:235-241: in CIRCULAR mode a spatial mask's crop is ignored and the whole
    grid runs, through propagate_vnn_2d and through the trainer's evaluation."""
    from neurocell import VNNParams, VNNTrainer, VonNeumannNetwork, adamw, propagate_vnn_2d
    from neurocell.topology import ChipTopology2D
    topo = ChipTopology2D.clp_chip(n=16, padding_mode="CIRCULAR")
    H, W = topo.grid_shape
    rng = np.random.default_rng(23)
    cell = np.stack([rng.normal(0, 0.3, (H, W)), rng.normal(0, 0.1, (H, W)),
                     rng.normal(0, 1.0, (H, W))]).astype(np.float32)
    filt = rng.normal(0, 1.0 / 3.0, (1, 1, 3, 3)).astype(np.float32)
    x = (rng.random((8, 2)) > 0.5).astype(np.float32)
    p = VNNParams(dev(cell), dev(filt))
    full = propagate_vnn_2d(p, dev(x), topo)
    crop = propagate_vnn_2d(p, dev(x), topo, spatial_mask=mask((1, 10, 2, 12)))
    assert np.array_equal(host(full), host(crop))
    geom = O.Geometry((H, W), (3, 3), 1, 4, [("coords", list(topo.in_ports[0].coords))],
                      ("coords", list(topo.out_port.coords)), padding_mode="CIRCULAR")
    assert rel_l2(host(full), O.propagate(cell, filt, x, geom)[0]) < FWD_TOL
    model = VonNeumannNetwork(topo)
    tr = VNNTrainer(model.apply, adamw(0.01), batch_size=8)
    y = dev(rng.integers(0, 2, size=(1,) + tuple(full.shape)).astype(np.float32))
    m_full = tr.evaluate_metric(p, dev(x[None]), y)
    m_crop = tr.evaluate_metric_adaptive(p, dev(x[None]), y, mask((1, 10, 2, 12)))
    assert float(m_full) == float(m_crop)


@pytest.mark.parametrize("mode,bbox", [("continuous", None), ("ste_ternary", CROP),
                                       ("annealed", None)])
def test_precompute_step_params_autograd(mode, bbox):
    from neurocell import precompute_step_params, VNNParams
    from neurocell.topology import ChipTopology2D
    geom, cell, filt, _, _ = alu_case(5, B=1)
    topo = ChipTopology2D.alu_chip(out_width=2)
    ct = dev(cell).requires_grad_()
    sp = precompute_step_params(VNNParams(ct, dev(filt)), topo, roi_bbox=bbox, codd_mode=mode,
                                state_temperature=0.3)
    ref = O.precompute_step_params(cell, geom, roi_bbox=bbox, mode=mode, tau=0.3)
    rng = np.random.default_rng(6)
    keys = ("w_eff_roi", "s_eff_roi", "b_roi", "w_eff_out", "s_eff_out", "b_out")
    grads = {k: rng.normal(size=ref[k].shape) for k in keys}
    loss = 0
    for k in keys:
        assert rel_l2(host(getattr(sp, k)), ref[k]) < FWD_TOL, k
        loss = loss + (getattr(sp, k) * dev(grads[k].astype(np.float32))).sum()
    assert rel_l2(host(sp.s_prob), ref["s_prob"]) < FWD_TOL
    loss.backward()
    r_g = O.precompute_step_params_vjp(cell, geom, grads, roi_bbox=bbox, mode=mode, tau=0.3)
    assert rel_l2(host(ct.grad), r_g) < GRAD_TOL


@pytest.mark.parametrize("mode", ["continuous", "annealed", "ste_binary", "ste_ternary"])
def test_codd_state_probs_autograd(mode):
    from neurocell import compute_codd_state_probs
    geom, cell, _, _, _ = alu_case(7, B=1)
    s = dev(cell[2]).requires_grad_()
    p = compute_codd_state_probs(s, geom.io_state_mask, codd_mode=mode, state_temperature=0.5)
    g = np.random.default_rng(8).normal(size=p.shape).astype(np.float32)
    p.backward(dev(g))
    rp, rd = O.codd_state_probs(cell[2], geom.io_state_mask, mode=mode, tau=0.5)
    assert rel_l2(host(p), rp) < FWD_TOL
    assert rel_l2(host(s.grad), rd * g) < GRAD_TOL


# ------------------------------------------------------------------ propagation

@pytest.mark.parametrize("mode,tau,bbox", [("continuous", 1.0, None), ("ste_ternary", 0.1, CROP)])
def test_propagate_autograd(mode, tau, bbox):
    from neurocell import VNNParams, propagate_vnn_2d
    from neurocell.topology import ChipTopology2D
    geom, cell, filt, x, _ = alu_case(9, B=8)
    topo = ChipTopology2D.alu_chip(out_width=2)
    p = VNNParams(dev(cell).requires_grad_(), dev(filt).requires_grad_())
    out = propagate_vnn_2d(p, dev(x), topo, codd_mode=mode, state_temperature=tau,
                           spatial_mask=mask(bbox))
    g = np.random.default_rng(10).normal(size=tuple(out.shape)).astype(np.float32)
    out.backward(dev(g))
    r_out, r_gc, r_gf = O.propagate_vjp(cell, filt, x, geom, g, roi_bbox=bbox, mode=mode,
                                        tau=tau)
    assert rel_l2(host(out), r_out) < FWD_TOL
    assert rel_l2(host(p.cell_params.grad), r_gc) < GRAD_TOL
    assert rel_l2(host(p.greens_filters.grad), r_gf) < GRAD_TOL


@pytest.mark.parametrize("bbox,use_univ", [(None, True), (CROP, True), (None, False)])
def test_return_universe_autograd(bbox, use_univ):
    """propagate_vnn_2d(..., return_universe=True) on the ALU chip (unit_vnn_alu_parity.py:
    76-100): the port equals the stateless call's, the universe is the oracle's final cells,
    and autograd through either output reaches the parameters."""
    from neurocell import VNNParams, propagate_vnn_2d
    from neurocell.topology import ChipTopology2D
    geom, cell, filt, x, _ = alu_case(12, B=8)
    topo = ChipTopology2D.alu_chip(out_width=2)
    p = VNNParams(dev(cell).requires_grad_(), dev(filt).requires_grad_())
    kw = dict(spatial_mask=mask(bbox), final_activate="sigmoid")
    out, univ = propagate_vnn_2d(p, dev(x), topo, return_universe=True, **kw)
    with torch.no_grad():
        plain = propagate_vnn_2d(p, dev(x), topo, **kw)
    rng = np.random.default_rng(13)
    g = rng.normal(size=tuple(out.shape)).astype(np.float32)
    gu = rng.normal(size=tuple(univ.shape)).astype(np.float32) if use_univ else None
    loss = (out * dev(g)).sum() + ((univ * dev(gu)).sum() if use_univ else 0.0)
    loss.backward()
    ok = dict(roi_bbox=bbox, final_act="sigmoid", universe=True)
    r_out, r_c = O.propagate(cell, filt, x, geom, **ok)
    _, r_gc, r_gf = O.propagate_vjp(cell, filt, x, geom, g, g_universe=gu, fwd=(r_out, r_c), **ok)
    assert rel_l2(host(out), r_out) < FWD_TOL
    assert rel_l2(host(plain), host(out)) < FWD_TOL
    assert rel_l2(host(univ), r_c["universe"]) < FWD_TOL
    assert rel_l2(host(p.cell_params.grad), r_gc) < GRAD_TOL
    assert rel_l2(host(p.greens_filters.grad), r_gf) < GRAD_TOL


def test_two_live_graphs():
    """Two forwards kept alive before their backwards (each call owns its activations)."""
    from neurocell import VNNParams, propagate_vnn_2d
    from neurocell.topology import ChipTopology2D
    geom, cell, filt, x, _ = alu_case(11, B=8)
    topo = ChipTopology2D.alu_chip(out_width=2)
    p = VNNParams(dev(cell).requires_grad_(), dev(filt).requires_grad_())
    o1 = propagate_vnn_2d(p, dev(x[:4].copy()), topo)
    o2 = propagate_vnn_2d(p, dev(x[4:].copy()), topo)
    (o1.sum() + 2.0 * o2.sum()).backward()
    g = np.ones((8,) + geom.out_size, np.float32)
    g[4:] = 2.0
    _, r_gc, r_gf = O.propagate_vjp(cell, filt, x, geom, g)
    assert rel_l2(host(p.cell_params.grad), r_gc) < GRAD_TOL
    assert rel_l2(host(p.greens_filters.grad), r_gf) < GRAD_TOL


# ------------------------------------------------------------------ model

def test_model_checkpoint_and_states(tmp_path):
    from neurocell import VonNeumannNetwork
    from neurocell.topology import ChipTopology2D
    geom, _, _, x, _ = alu_case(12, B=4)
    topo = ChipTopology2D.alu_chip(out_width=2)
    model = VonNeumannNetwork(topo, codd_mode="ste_ternary", state_temperature=0.2)
    params = model.init(42)
    assert params.cell_params.shape == (3, 62, 62) and params.greens_filters.shape == (16, 1, 23, 13)
    f = tmp_path / "ck.npz"
    model.save_checkpoint(str(f), params, note=np.int32(7))
    back = VonNeumannNetwork.load_checkpoint(str(f))
    assert torch.equal(back.cell_params, params.cell_params)
    assert torch.equal(back.greens_filters, params.greens_filters)
    cell, filt = host(params.cell_params), host(params.greens_filters)
    out = model.apply(params, dev(x))
    r_out, _ = O.propagate(cell, filt, x, geom, mode="ste_ternary", tau=0.2)
    assert rel_l2(host(out), r_out) < FWD_TOL
    s = model.effective_states(params)
    r_s, _ = O.codd_state_probs(cell[2], geom.io_state_mask, mode="ste_ternary", tau=0.2)
    assert rel_l2(host(s), r_s) < FWD_TOL
    th = host(VonNeumannNetwork.threshold_states(params.states))
    sr = cell[2]
    ref = np.where(sr >= 0.6, 2.0, sr)
    ref = np.where((ref > 0) & (ref < 0.6), 1.0, ref)
    assert np.array_equal(th, ref.astype(np.float32))


# ------------------------------------------------------------------ trainer

def _oracle_steps(cell, filt, xs, ys, geom, lr, n, bbox=None, mode="continuous", tau=1.0,
                  **kw):
    p = np.concatenate([cell.ravel(), filt.ravel()]).astype(np.float64)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    nc = cell.size
    losses = []
    for i in range(n):
        c = p[:nc].reshape(cell.shape).astype(np.float32)
        f = p[nc:].reshape(filt.shape).astype(np.float32)
        out, _ = O.propagate(c, f, xs[i], geom, roi_bbox=bbox, mode=mode, tau=tau, **kw)
        loss, g_out = O.mse_loss(out, ys[i])
        _, gc, gf = O.propagate_vjp(c, f, xs[i], geom, g_out, roi_bbox=bbox, mode=mode, tau=tau,
                                    **kw)
        g = np.concatenate([gc.ravel(), gf.ravel()])
        p, m, v, _ = O.adamw_step(p, g, m, v, i, lr(i) if callable(lr) else lr)
        losses.append(loss)
    return p[:nc].reshape(cell.shape), p[nc:].reshape(filt.shape), np.array(losses)


def _trainer_case(seed, nb, B=8, out_width=2):
    from neurocell.topology import ChipTopology2D
    geom, cell, filt, _, _ = alu_case(seed, B=1, out_width=out_width)
    xs, ys = [], []
    for i in range(nb):
        _, _, _, x, y = alu_case(seed * 100 + i, B=B, out_width=out_width)
        xs.append(x)
        ys.append(y)
    return geom, ChipTopology2D.alu_chip(out_width=out_width), cell, filt, np.stack(xs), \
        np.stack(ys)


@pytest.mark.parametrize("variant", ["plain", "adaptive", "annealed"])
def test_trainer_steps_vs_oracle(variant):
    from neurocell import VNNParams, VNNTrainer, VonNeumannNetwork, adamw
    from neurocell import warmup_cosine_decay_schedule as wcd
    geom, topo, cell, filt, xs, ys = _trainer_case(13, nb=2)
    sched = wcd(0.001, 0.03, 1, 10, 0.0005)
    model = VonNeumannNetwork(topo)
    tr = VNNTrainer(model.apply, adamw(sched), batch_size=8)
    params = VNNParams(dev(cell), dev(filt))
    state = tr.optimizer.init(params)
    bbox, mode, tau = None, "continuous", 1.0
    losses = []
    for i in range(2):
        if variant == "plain":
            params, state, loss = tr.train_step(params, state, dev(xs[i]), dev(ys[i]))
        elif variant == "adaptive":
            bbox = CROP
            params, state, loss = tr.train_step_adaptive(params, state, dev(xs[i]), dev(ys[i]),
                                                         mask(bbox))
        else:
            mode, tau = "ste_ternary", 0.5
            params, state, loss = tr.train_step_annealed(params, state, dev(xs[i]), dev(ys[i]),
                                                         state_temperature=tau, codd_mode=mode)
        losses.append(float(loss))
    r_c, r_f, r_l = _oracle_steps(cell, filt, xs, ys, geom, sched, 2, bbox, mode, tau)
    assert rel_l2(losses, r_l) < FWD_TOL
    assert rel_l2(host(params.cell_params) - cell, r_c - cell) < TRAJ_TOL
    assert rel_l2(host(params.greens_filters) - filt, r_f - filt) < TRAJ_TOL
    assert int(state.count.item()) == 2


def test_trainer_gol_valid_universe_port():
    """Training VALID Game of Life (topology.py:359-388): its universe port lies on the border,
    so every step reads the port from the final universe (propagator.py:684-734)."""
    from neurocell import VNNParams, VNNTrainer, VonNeumannNetwork, adamw
    from neurocell.topology import ChipTopology2D
    n, M = 16, 4
    topo = ChipTopology2D.gol_chip(n=n, kernel_size=(3, 3), directions=M, depth=3)
    geom = O.Geometry((n, n), (3, 3), M, 3, [("rect", (0, 0), (n, n))], ("rect", (0, 0), (n, n)))
    rng = np.random.default_rng(41)
    cell = np.stack([rng.normal(0, 0.1, (n, n)), rng.normal(0, 0.2, (n, n)),
                     rng.normal(0, 1.0, (n, n))]).astype(np.float32)
    filt = rng.normal(0, 1.0 / 3.0, (M, 1, 3, 3)).astype(np.float32)
    xs = (rng.random((2, 4, n, n)) > 0.5).astype(np.float32)
    ys = (rng.random((2, 4, n, n)) > 0.5).astype(np.float32)
    tr = VNNTrainer(VonNeumannNetwork(topo, final_activate="sigmoid").apply, adamw(0.01),
                    batch_size=4)
    params = VNNParams(dev(cell), dev(filt))
    state = tr.optimizer.init(params)
    losses = []
    for i in range(2):
        params, state, loss = tr.train_step(params, state, dev(xs[i]), dev(ys[i]))
        losses.append(float(loss))
    r_c, r_f, r_l = _oracle_steps(cell, filt, xs, ys, geom, 0.01, 2, final_act="sigmoid",
                                  universe=True)
    assert rel_l2(losses, r_l) < FWD_TOL
    assert rel_l2(host(params.cell_params) - cell, r_c - cell) < TRAJ_TOL
    assert rel_l2(host(params.greens_filters) - filt, r_f - filt) < TRAJ_TOL


def test_trainer_graph_replay_matches_eager():
    """Epoch graphs (first call eager, second captured, later replayed) against a trainer that
    always launches eagerly: bit-identical parameters, moments and losses, with eager work and
    synchronisations between replays."""
    from neurocell import VNNParams, VNNTrainer, VonNeumannNetwork, adamw
    _, topo, cell, filt, xs, ys = _trainer_case(14, nb=3)
    model = VonNeumannNetwork(topo)
    res = []
    for use_graphs in (True, False):
        tr = VNNTrainer(model.apply, adamw(0.01), batch_size=8, use_graphs=use_graphs)
        params = VNNParams(dev(cell), dev(filt))
        state = tr.optimizer.init(params)
        x, y = dev(xs), dev(ys)
        ep = []
        for e in range(4):
            params, state, loss = tr.train_epoch(params, state, x, y)
            torch.cuda.synchronize()
            ep.append(float(loss))
            _ = torch.ones(1000, device="cuda").sum()  # unrelated eager work between replays
        res.append((host(params.cell_params), host(params.greens_filters),
                    host(state.mu.cell_params), np.array(ep)))
    for a, b in zip(*res):
        assert np.array_equal(a, b)


def test_trainer_generic_path_matches_fused():
    from neurocell import (VNNParams, VNNTrainer, VonNeumannNetwork, adamw, default_mse_loss)
    _, topo, cell, filt, xs, ys = _trainer_case(15, nb=2)
    model = VonNeumannNetwork(topo)
    outs = []
    for loss_fn in (None, default_mse_loss):
        tr = VNNTrainer(model.apply, adamw(0.01), batch_size=8, loss_fn=loss_fn)
        assert tr.fused == (loss_fn is None)
        params = VNNParams(dev(cell), dev(filt))
        state = tr.optimizer.init(params)
        params, state, loss = tr.train_epoch(params, state, dev(xs), dev(ys))
        outs.append((host(params.cell_params), host(params.greens_filters), float(loss)))
    (c0, f0, l0), (c1, f1, l1) = outs
    assert abs(l0 - l1) <= 1e-5 * abs(l1)
    assert rel_l2(c0 - cell, c1 - cell) < TRAJ_TOL
    assert rel_l2(f0 - filt, f1 - filt) < TRAJ_TOL


def test_evaluate_packed_and_metric():
    from neurocell import VNNParams, VNNTrainer, VonNeumannNetwork, adamw
    geom, topo, cell, filt, xs, ys = _trainer_case(16, nb=2, out_width=1)
    model = VonNeumannNetwork(topo)
    tr = VNNTrainer(model.apply, adamw(0.01), batch_size=8)
    params = VNNParams(dev(cell), dev(filt))
    ref_out = np.stack([O.propagate(cell, filt, xs[i], geom)[0] for i in range(2)])
    bits = np.clip(np.round(ref_out.reshape(2, 8, 8)), 0, 255).astype(np.int64)
    ref_pred = (bits * np.array([128, 64, 32, 16, 8, 4, 2, 1])).sum(-1) % 256
    rng = np.random.default_rng(17)
    y_packed = np.where(rng.random((2, 8)) < 0.5, ref_pred, rng.integers(0, 256, (2, 8)))
    y_packed = y_packed.astype(np.uint8)[..., None]
    acc, preds = tr.evaluate_packed(params, dev(xs), dev(y_packed))
    near_half = np.abs(np.abs(ref_out - np.round(ref_out)) - 0.5) < 1e-4
    ok = ~near_half.reshape(2, 8, 8).any(-1)
    assert np.array_equal(host(preds)[..., 0][ok], ref_pred[ok])
    hits = (host(preds) == y_packed).mean(axis=(1, 2))
    assert abs(float(acc) - float(hits.mean())) < 1e-6
    m = tr.evaluate_metric(params, dev(xs), dev(ys.reshape(2, 8, 8)))
    r_m = np.mean([(np.round(ref_out[i].reshape(8, 8)) == np.round(ys[i].reshape(8, 8))).mean()
                   for i in range(2)])
    assert abs(float(m) - r_m) < 1e-6


def test_train_epochs_runs():
    from neurocell import VNNParams, VNNTrainer, VonNeumannNetwork, adamw
    _, topo, cell, filt, xs, ys = _trainer_case(18, nb=3)
    model = VonNeumannNetwork(topo)
    tr = VNNTrainer(model.apply, adamw(0.01), batch_size=8)
    params = VNNParams(dev(cell), dev(filt))
    state = tr.optimizer.init(params)
    x = dev(xs.reshape(24, 3, 8, 1))
    y = dev(ys.reshape(24, 8, 2))
    params, state, losses = tr.train_epochs(params, state, x, y, rng=0, num_epochs=3)
    assert losses.shape == (3,) and torch.isfinite(losses).all()
    assert int(state.count.item()) == 9


def test_trained_checkpoint_alu_accuracy():
    """End to end on trained parameters: the reference's shipped ALU checkpoint evaluated on a
    generated ALU test split (datasets.py:133-179) with the packed-accuracy metric, its Codd
    states hardened as it was trained (ste_ternary, temperature 0.1).  The first batch's
    predictions must equal the float64 oracle's (bytes whose bits sit within 1e-4 of a
    rounding tie excepted), and the accuracy must be that of the trained ALU (the reference's
    README quotes 98.35% test accuracy after 30 epochs).  In continuous mode the same
    parameters score about 87%: they were trained with hardened states."""
    import os
    from neurocell import (VNNTrainer, VonNeumannNetwork, adamw, prepare_alu_device_dataset)
    from neurocell.topology import ChipTopology2D
    path = os.path.join(os.path.dirname(__file__), "golden", "alu_arithmetic_cells.npz")
    params = VonNeumannNetwork.load_checkpoint(path)
    np.random.seed(2026)
    ds = prepare_alu_device_dataset(samples=12800, batch_size=128)
    model = VonNeumannNetwork(ChipTopology2D.alu_chip(), codd_mode="ste_ternary",
                              state_temperature=0.1)
    tr = VNNTrainer(model.apply, adamw(0.01), batch_size=128)
    acc, preds = tr.evaluate_packed(params, ds.x_test, ds.y_test_packed)
    acc = float(acc)
    print(f"trained checkpoint: packed accuracy {acc:.6f} on {ds.x_test.shape[0] * 128} samples")
    geom = O.alu_geometry(out_width=1)
    x0 = host(ds.x_test[0])
    out = O.propagate(host(params.cell_params), host(params.greens_filters), x0, geom,
                      mode="ste_ternary", tau=0.1)[0]
    out = out.reshape(128, 8)
    bits = np.clip(np.round(out), 0, 255).astype(np.int64)
    ref = (bits * np.array([128, 64, 32, 16, 8, 4, 2, 1])).sum(-1) % 256
    ok = ~(np.abs(np.abs(out - np.round(out)) - 0.5) < 1e-4).any(-1)
    assert np.array_equal(host(preds[0])[:, 0][ok], ref[ok])
    assert acc >= 0.98, acc


def test_gated_filters_autograd():
    """gated_filters (propagator.py:266-267): the steps use sigmoid(filters).  Against the
    oracle run on the gated filters, with the raw filters' gradient by the chain rule through
    the sigmoid."""
    from neurocell import VNNParams, propagate_vnn_2d
    from neurocell.topology import ChipTopology2D
    geom, cell, filt, x, _ = alu_case(12, B=8)
    filt = (filt * 8.0).astype(np.float32)  # spread the gate over its range
    topo = ChipTopology2D.alu_chip(out_width=2)
    p = VNNParams(dev(cell).requires_grad_(), dev(filt).requires_grad_())
    out = propagate_vnn_2d(p, dev(x), topo, gated_filters=True)
    g = np.random.default_rng(13).normal(size=tuple(out.shape)).astype(np.float32)
    out.backward(dev(g))
    sg = 1.0 / (1.0 + np.exp(-filt.astype(np.float64)))
    r_out, r_gc, r_gf = O.propagate_vjp(cell, sg, x, geom, g)
    assert rel_l2(host(out), r_out) < FWD_TOL
    assert rel_l2(host(p.cell_params.grad), r_gc) < GRAD_TOL
    assert rel_l2(host(p.greens_filters.grad), r_gf * sg * (1.0 - sg)) < GRAD_TOL


def test_sharpen_autograd():
    """The weight-sharpening pre-filter (model.py:65-67, params.py:246-247) through the model
    API: the oracle runs on the weights sharpened by scipy's SAME correlation with the
    stencil, and the weights' gradient comes back through scipy's SAME convolution (the
    correlation's adjoint for an odd stencil)."""
    import scipy.signal
    from neurocell import VNNParams, VonNeumannNetwork
    from neurocell.model import sharpen_kernel
    from neurocell.topology import ChipTopology2D
    geom, cell, filt, x, _ = alu_case(14, B=8)
    topo = ChipTopology2D.alu_chip(out_width=2)
    model = VonNeumannNetwork(topo, sharpen=True)
    p = VNNParams(dev(cell).requires_grad_(), dev(filt).requires_grad_())
    out = model.apply(p, dev(x))
    g = np.random.default_rng(15).normal(size=tuple(out.shape)).astype(np.float32)
    out.backward(dev(g))
    k = sharpen_kernel().astype(np.float64)
    cell_s = cell.astype(np.float64).copy()
    cell_s[0] = scipy.signal.correlate2d(cell_s[0], k, mode="same")
    r_out, r_gc, r_gf = O.propagate_vjp(cell_s, filt, x, geom, g)
    g_w = scipy.signal.convolve2d(r_gc[0], k, mode="same")
    gc = host(p.cell_params.grad)
    assert rel_l2(host(out), r_out) < FWD_TOL
    assert rel_l2(gc[0], g_w) < GRAD_TOL
    assert rel_l2(gc[1:], r_gc[1:]) < GRAD_TOL
    assert rel_l2(host(p.greens_filters.grad), r_gf) < GRAD_TOL

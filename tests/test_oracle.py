"""Pins the float64 oracle (oracle/vnn_oracle.py) before it is trusted as the parity checker.

Each function of the oracle is checked against something it does not restate: the
reference's stored checkpoint (a trained 8-bit ALU must still compute its truth table), the
reference tests' known answers (topology numbers, Codd value sets, the zero thresholding gap,
the annealing endpoints, the factored == unfactored identity, the 32x32 adaptive bucket),
library routines (scipy correlate2d, torch float64 conv2d / layer_norm autograd), brute-force
restatements (the full-grid border theorem) and finite differences.  A plausible slip -- a
dropped term, a flipped kernel, a transposed operand, a wrong sign -- fails at least one.
"""
import math

import numpy as np
import pytest
import scipy.signal
import torch
import torch.nn.functional as F

from oracle import vnn_oracle as O

RNG = np.random.default_rng(1234)
ACTS = ("tanh", "sigmoid", "relu", "leaky_relu", "gelu", "identity")


def small_geometry(depth=3, M=3, kernel=(5, 3), grid=(16, 14), out=("rect", (6, 9), (3, 1))):
    return O.Geometry(grid, kernel, M, depth, [("rect", (5, 3), (4, 1)), ("rect", (4, 5), (1, 3))],
                      out)


def rand_cell(geom, rng, s_scale=1.0):
    H, W = geom.grid_shape
    return np.stack([rng.normal(0, 0.3, (H, W)), rng.normal(0, 0.2, (H, W)),
                     rng.normal(0, s_scale, (H, W))])


def rand_inputs(geom, B, rng):
    return [rng.normal(size=(B,) + tuple(p[2])) for p in geom.in_ports]


def torch_act(x, name):
    return {"tanh": torch.tanh, "sigmoid": torch.sigmoid, "relu": torch.relu,
            "leaky_relu": lambda v: F.leaky_relu(v, 0.01),
            "gelu": lambda v: F.gelu(v, approximate="tanh"), "identity": lambda v: v}[name](x)


# ------------------------------------------------------------------ golden fixture

def _alu_samples(B, seed=0):
    """The ALU truth table of datasets.py:77-130 (noise-free operands)."""
    rng = np.random.default_rng(seed)
    num = rng.integers(1, 128, B).astype(np.uint8)
    opr = rng.integers(1, 128, B).astype(np.uint8)
    ctl = rng.integers(1, 16, B).astype(np.uint8)
    one = np.uint8(1)
    conds = [(ctl == 0) | (ctl == 4), ctl == 1, (ctl == 2) | (ctl == 8), ctl == 3, ctl == 5,
             ctl == 6, ctl == 7]
    choices = [num, num + one, num + opr, num + opr + one, num - one, num - opr, num - opr - one]
    y = np.select(conds, [c.astype(np.uint8) for c in choices], default=num).astype(np.uint8)
    bits = lambda v: np.unpackbits(v[:, None], axis=1)
    x = np.stack([bits(num), bits(opr), bits(ctl)], 1).astype(np.float32)[..., None]
    return x, y


def test_trained_alu_checkpoint_computes_its_truth_table():
    """The reference's trained checkpoint (alu_arithmetic_cells.npz, README: 98.35% test
    accuracy) run through the oracle's pure-ROI forward must still be an 8-bit ALU; any
    mistake in injection, correlation orientation, standardisation, Codd gating or the port
    readout collapses the byte accuracy."""
    d = np.load("tests/golden/alu_arithmetic_cells.npz", allow_pickle=False)
    geom = O.alu_geometry(out_width=1)
    assert tuple(d["input_offset_x1"]) == geom.in_ports[0][1]
    assert tuple(d["input_offset_x2"]) == geom.in_ports[1][1]
    assert tuple(d["ctrl_offset"]) == geom.in_ports[2][1]
    assert tuple(d["ctrl_size"]) == tuple(geom.in_ports[2][2])
    assert tuple(d["output_offset"]) == geom.out_port[1]
    cell = np.stack([d["weights"], d["biases"], d["states"]]).astype(np.float32)
    filt = np.transpose(d["filters"], (3, 0, 1, 2)).astype(np.float32)
    x, y = _alu_samples(128)
    out, _ = O.propagate(cell, filt, x, geom, mode="ste_ternary", tau=0.1)
    pred = np.packbits(np.clip(np.round(out[..., 0]), 0, 1).astype(np.uint8), axis=1)[:, 0]
    assert (pred == y).mean() >= 0.95


# ------------------------------------------------------------------ topology known answers

def test_alu_geometry_known_answers():
    """unit_topology.py:24-81."""
    g = O.alu_geometry()
    assert g.grid_shape == (62, 62)
    assert (g.pad_h, g.pad_w) == (11, 6)
    assert g.roi_shape == (40, 50)
    assert g.fft_shape == (64, 64)
    assert g.in_ports[0][1:] == ((23, 23), (8, 1))
    assert g.in_ports[1][1:] == ((32, 23), (8, 1))
    assert g.in_ports[2][1:] == ((18, 28), (1, 8))
    assert g.out_port[1:] == ((27, 41), (8, 1))
    rows, cols = g.out_cells_roi
    assert (rows[0], cols[0]) == (16, 35)
    assert int(g.io_state_mask.sum()) == 32
    assert int(g.out_weight_mask.sum()) == 8
    with pytest.raises(ValueError):
        O.Geometry((62, 62), (22, 13), 16, 4, [], ("rect", (27, 41), (8, 1)))


def test_inject_column_quirk():
    """propagator.py:124-130: a 3-D (B, ih, iw) per-port input is written with its own shape,
    so the ALU driver's (B,3,8,1) ctrl lands as an 8x1 column at grid (18,28)."""
    g = O.alu_geometry()
    x = np.zeros((1, 3, 8, 1))
    x[0, 2, :, 0] = np.arange(1, 9)
    roi = O.inject_inputs_roi(O.split_ports(x, g), g)
    col = roi[0, 18 - 11:18 - 11 + 8, 28 - 6]
    assert np.array_equal(col, np.arange(1, 9))


# ------------------------------------------------------------------ correlation

def test_direct_correlation_matches_scipy():
    x = RNG.normal(size=(2, 11, 9))
    g = RNG.normal(size=(3, 5, 3))
    z = O.conv2d_direct(x, g, (2, 1))
    for b in range(2):
        xp = np.pad(x[b], ((2, 2), (1, 1)))
        for m in range(3):
            np.testing.assert_allclose(z[b, m], scipy.signal.correlate2d(xp, g[m], "valid"),
                                       rtol=0, atol=1e-12)


@pytest.mark.parametrize("shape", [((2, 40, 50), (4, 23, 13), (64, 64)),
                                   ((3, 10, 12), (2, 5, 3), (16, 16)),
                                   ((2, 20, 50), (3, 9, 13), (32, 64))])
def test_fft_correlation_matches_direct(shape):
    (B, h, w), (M, kh, kw), fs = shape
    x = RNG.normal(size=(B, h, w))
    g = RNG.normal(size=(M, 1, kh, kw))
    pad = ((kh - 1) // 2, (kw - 1) // 2)
    z, _ = O.conv2d_fft(x, g[:, 0], pad, (h, w), fs)
    np.testing.assert_allclose(z, O.conv2d_direct(x, g[:, 0], pad), rtol=0, atol=1e-10)
    # VALID form (the hoisted border conv): shift kh-1, kw-1
    hv, wv = h - kh + 1, w - kw + 1
    if hv > 0 and wv > 0:
        zv, _ = O.conv2d_fft(x, g[:, 0], (kh - 1, kw - 1), (hv, wv), fs)
        np.testing.assert_allclose(zv, O.conv2d_direct(x, g[:, 0], (0, 0)), rtol=0, atol=1e-10)


def test_direct_backward_matches_torch_autograd():
    x = RNG.normal(size=(2, 12, 10))
    g = RNG.normal(size=(3, 5, 3))
    gz = RNG.normal(size=(2, 3, 12, 10))
    dx, dg = O.conv2d_bwd_direct(gz, x, g, (2, 1))
    xt = torch.tensor(x[:, None], requires_grad=True)
    gt = torch.tensor(g[:, None], requires_grad=True)
    F.conv2d(xt, gt, padding=(2, 1)).backward(torch.tensor(gz))
    np.testing.assert_allclose(dx, xt.grad[:, 0].numpy(), rtol=0, atol=1e-10)
    np.testing.assert_allclose(dg, gt.grad[:, 0].numpy(), rtol=0, atol=1e-10)


@pytest.mark.parametrize("shape", [((2, 40, 50), (3, 23, 13), (64, 64)),
                                   ((2, 24, 32), (2, 23, 13), (64, 64)),
                                   ((3, 10, 12), (2, 5, 3), (16, 16))])
def test_unshifted_plancherel_backward_matches_direct(shape):
    (B, h, w), (M, kh, kw), fs = shape
    x = RNG.normal(size=(B, h, w))
    g = RNG.normal(size=(M, kh, kw))
    gz = RNG.normal(size=(B, M, h, w))
    pad = ((kh - 1) // 2, (kw - 1) // 2)
    dx, dGh = O.conv2d_fft_unshifted_bwd(gz, x, g, pad, fs)
    dg = O.filter_grad_from_unshifted(dGh, (kh, kw), pad, fs)
    r_dx, r_dg = O.conv2d_bwd_direct(gz, x, g, pad)
    np.testing.assert_allclose(dx, r_dx, rtol=0, atol=1e-9)
    np.testing.assert_allclose(dg, r_dg, rtol=0, atol=1e-9)


# ------------------------------------------------------------------ epilogues

def _torch_epilogue(z, d, w, s, b, act, hb):
    zt = z + d if hb else z
    zn = F.layer_norm(zt, zt.shape[-2:], eps=1e-5)
    return w * zn.sum(1) + s * torch_act(zn + b, act).sum(1)


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("hb", [True, False])
def test_epilogue_matches_torch_layer_norm_autograd(act, hb):
    B, M, h, w = 3, 4, 7, 9
    z, d = RNG.normal(size=(B, M, h, w)), RNG.normal(size=(1, M, h, w))
    wt, st, bt = (RNG.normal(size=(h, w)) for _ in range(3))
    gy = RNG.normal(size=(B, h, w))
    out, mean, rstd = O.epilogue_fwd(z, d, wt, st, bt, act, hb)
    gz, gdb, gw, gs, gb = O.epilogue_bwd(z, d, wt, st, bt, mean, rstd, gy, act, hb)
    ts = [torch.tensor(a, requires_grad=True) for a in (z, d, wt, st, bt)]
    ref = _torch_epilogue(*ts, act, hb)
    ref.backward(torch.tensor(gy))
    np.testing.assert_allclose(out, ref.detach().numpy(), rtol=1e-10, atol=1e-10)
    refs = [ts[0].grad, ts[1].grad[0] if hb else torch.zeros(M, h, w), ts[2].grad, ts[3].grad,
            ts[4].grad]
    for mine, r in zip((gz, gdb, gw, gs, gb), refs):
        np.testing.assert_allclose(mine, r.numpy(), rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("final_act", [None, "tanh", "sigmoid"])
@pytest.mark.parametrize("coords", [False, True])
def test_port_epilogue_matches_torch_autograd(final_act, coords):
    B, M, h, w = 3, 4, 8, 10
    if coords:
        rows, cols, size = np.array([1, 5, 5, 7]), np.array([2, 3, 3, 9]), (4, 1)
    else:
        rr, cc = np.meshgrid(np.arange(3, 6), np.arange(4, 6), indexing="ij")
        rows, cols, size = rr.ravel(), cc.ravel(), (3, 2)
    z, d = RNG.normal(size=(B, M, h, w)), RNG.normal(size=(1, M, h, w))
    wo, so, bo = (RNG.normal(size=size) for _ in range(3))
    g_out = RNG.normal(size=(B,) + size)
    out, aux = O.port_fwd(z, d, rows, cols, size, wo, so, bo, True, final_act)
    gz, gdb, gw, gs, gb = O.port_bwd(z, d, rows, cols, size, wo, so, bo, aux, g_out, True,
                                     final_act)
    ts = [torch.tensor(a, requires_grad=True) for a in (z, d, wo, so, bo)]
    zn = F.layer_norm(ts[0] + ts[1], (h, w), eps=1e-5)
    zo = zn[:, :, torch.tensor(rows), torch.tensor(cols)].reshape(B, M, *size)
    if final_act is None:  # identity gating: (w+s)*sum z + M*s*b (kernels_pallas.py:1538-1551)
        ref = (ts[2] + ts[3]) * zo.sum(1) + M * ts[3] * ts[4]
    else:
        ref = torch_act(ts[2] * zo.sum(1) + ts[3] * torch_act(zo + ts[4], final_act).sum(1),
                        final_act)
    ref.backward(torch.tensor(g_out))
    np.testing.assert_allclose(out, ref.detach().numpy(), rtol=1e-10, atol=1e-10)
    for mine, r in zip((gz, gdb, gw, gs, gb), (ts[0].grad, ts[1].grad[0], ts[2].grad,
                                               ts[3].grad, ts[4].grad)):
        np.testing.assert_allclose(mine, r.numpy(), rtol=1e-9, atol=1e-9)


# ------------------------------------------------------------------ Codd fusion

def test_codd_value_sets_and_pins():
    """unit_milestone8_pallas_and_codd.py:207-237 value sets; pinned IO cells are 1 with zero
    derivative; continuous derivative against central differences."""
    g = O.alu_geometry()
    s = np.random.default_rng(5).uniform(-1.0, 1.2, g.grid_shape)
    assert O.CODD_MODES == ("continuous", "annealed", "ste_binary", "ste_ternary")
    pb, _ = O.codd_state_probs(s, g.io_state_mask, mode="ste_binary", tau=0.3)
    assert set(np.unique(pb)) <= {0.0, 1.0}
    pt, _ = O.codd_state_probs(s, g.io_state_mask, mode="ste_ternary", tau=0.3)
    assert set(np.unique(pt)) <= {0.0, 0.5, 1.0}
    io = g.io_state_mask
    for mode in O.CODD_MODES:
        # params.py:58, 77-78: IO cells read S = 1 (hard_pin_io instead forces p = 1);
        # either way p is constant there
        p, dp = O.codd_state_probs(s, io, False, mode, 0.3)
        p1, _ = O.codd_state_probs(np.ones_like(s), np.zeros_like(io), False, mode, 0.3)
        assert np.array_equal(p[io], p1[io]) and np.all(dp[io] == 0.0)
        p, dp = O.codd_state_probs(s, io, True, mode, 0.3)
        assert np.all(p[io] == 1.0) and np.all(dp[io] == 0.0)
    p, dp = O.codd_state_probs(s, g.io_state_mask, mode="continuous")
    e = 1e-6
    fd = (O.codd_state_probs(s + e, g.io_state_mask)[0]
          - O.codd_state_probs(s - e, g.io_state_mask)[0]) / (2 * e)
    np.testing.assert_allclose(dp, np.where(g.io_state_mask, 0.0, fd), atol=1e-8)
    # straight-through: the STE modes carry the annealed (soft) derivative
    _, da = O.codd_state_probs(s, g.io_state_mask, mode="annealed", tau=0.3)
    for mode in ("ste_binary", "ste_ternary"):
        assert np.array_equal(O.codd_state_probs(s, g.io_state_mask, mode=mode, tau=0.3)[1], da)


def test_factored_equals_unfactored():
    """unit_params.py:102-134: w_eff*sum_m z + s_eff*sum_m tanh(z+b) equals the legacy
    mean_m(z*w*(1-s) + tanh(z+b)*s) on the ROI."""
    g = O.alu_geometry()
    cell = rand_cell(g, np.random.default_rng(6))
    sp = O.precompute_step_params(cell, g)
    z = np.random.default_rng(7).normal(size=(2, 16, 40, 50))
    rh, rw = g.pad_h, g.pad_w
    roi = (slice(rh, 62 - rh), slice(rw, 62 - rw))
    legacy = np.mean(z * (sp["w_pinned"][roi] * (1 - sp["s_prob"][roi]))
                     + np.tanh(z + sp["b_full"][roi]) * sp["s_prob"][roi], axis=1)
    fused = sp["w_eff_roi"] * z.sum(1) + sp["s_eff_roi"] * np.tanh(z + sp["b_roi"]).sum(1)
    assert np.max(np.abs(legacy - fused)) < 1e-12


@pytest.mark.parametrize("mode,bbox", [("continuous", None), ("annealed", (3, 30, 8, 44)),
                                       ("continuous", (6, 30, 10, 42))])
def test_precompute_vjp_matches_finite_differences(mode, bbox):
    g = O.alu_geometry(out_width=2)
    rng = np.random.default_rng(8)
    cell = rand_cell(g, rng)
    ref = O.precompute_step_params(cell, g, roi_bbox=bbox, mode=mode, tau=0.4)
    keys = ("w_eff_roi", "s_eff_roi", "b_roi", "border_2d", "w_eff_out", "s_eff_out", "b_out")
    grads = {k: rng.normal(size=np.shape(ref[k])) for k in keys}
    gc = O.precompute_step_params_vjp(cell, g, grads, roi_bbox=bbox, mode=mode, tau=0.4)
    v = rng.normal(size=cell.shape)

    def L(c):
        sp = O.precompute_step_params(c, g, roi_bbox=bbox, mode=mode, tau=0.4)
        return sum(float((sp[k] * grads[k]).sum()) for k in keys)
    e = 1e-6
    fd = (L(cell + e * v) - L(cell - e * v)) / (2 * e)
    assert abs(fd - float((gc * v).sum())) <= 1e-6 * max(1.0, abs(fd))


# ------------------------------------------------------------------ whole step

@pytest.mark.parametrize("final_act,mode", [(None, "continuous"), ("tanh", "annealed"),
                                            (None, "ste_ternary")])
def test_border_theorem_pure_roi_equals_full_grid(final_act, mode):
    """propagator.py:1-9: the pure-ROI step plus the hoisted border conv reproduces the
    full-grid VALID propagation (contrib/forward.py:737-810) exactly."""
    g = small_geometry(depth=3)
    rng = np.random.default_rng(9)
    cell, filt = rand_cell(g, rng), rng.normal(size=(3, 1, 5, 3))
    x = rand_inputs(g, 2, rng)
    full = O.propagate_full_grid(cell, filt, x, g, final_act=final_act, mode=mode, tau=0.5)
    for conv in ("fft", "direct"):
        roi, _ = O.propagate(cell, filt, x, g, final_act=final_act, mode=mode, tau=0.5,
                             conv=conv)
        np.testing.assert_allclose(roi, full, rtol=0, atol=1e-10)


def test_border_theorem_alu():
    g = O.alu_geometry(out_width=2, directions=4)
    rng = np.random.default_rng(10)
    cell, filt = rand_cell(g, rng), rng.normal(0, 0.05, size=(4, 1, 23, 13))
    x = (rng.random((2, 3, 8, 1)) > 0.5).astype(float)
    roi, _ = O.propagate(cell, filt, x, g)
    np.testing.assert_allclose(roi, O.propagate_full_grid(cell, filt, x, g), rtol=0, atol=1e-10)


@pytest.mark.parametrize("final_act,mode,bbox,pin", [
    (None, "continuous", None, False), ("tanh", "annealed", None, True),
    (None, "continuous", (1, 10, 2, 10), False)])
def test_propagate_vjp_matches_finite_differences(final_act, mode, bbox, pin):
    g = small_geometry(depth=3)
    rng = np.random.default_rng(11)
    cell, filt = rand_cell(g, rng), rng.normal(size=(3, 1, 5, 3))
    x = rand_inputs(g, 2, rng)
    kw = dict(final_act=final_act, mode=mode, tau=0.7, roi_bbox=bbox, hard_pin_io=pin)
    out, _ = O.propagate(cell, filt, x, g, **kw)
    g_out = rng.normal(size=out.shape)
    _, gc, gf = O.propagate_vjp(cell, filt, x, g, g_out, **kw)
    vc, vf = rng.normal(size=cell.shape), rng.normal(size=filt.shape)

    def L(c, f):
        return float((O.propagate(c, f, x, g, **kw)[0] * g_out).sum())
    e = 1e-6
    fd = (L(cell + e * vc, filt + e * vf) - L(cell - e * vc, filt - e * vf)) / (2 * e)
    an = float((gc * vc).sum() + (gf * vf).sum())
    assert abs(fd - an) <= 1e-6 * max(1.0, abs(an))


BORDER_PORT = ("coords", [(0, 0), (1, 5), (8, 7), (15, 13), (6, 9)])


@pytest.mark.parametrize("final_act,out", [(None, None), ("tanh", None), ("sigmoid", BORDER_PORT),
                                           (None, ("rect", (0, 0), (16, 14)))])
def test_universe_equals_full_grid(final_act, out):
    """propagator.py:684-734 (return_universe / an output port on the border): the pure-ROI
    last step embedded with final_act(B) * s_prob around it is the full-grid VALID propagation
    (contrib/forward.py:737-810), universe and port alike (unit_vnn_alu_parity.py:76-100)."""
    g = small_geometry(depth=3) if out is None else small_geometry(depth=3, out=out)
    rng = np.random.default_rng(21)
    cell, filt = rand_cell(g, rng), rng.normal(size=(3, 1, 5, 3))
    x = rand_inputs(g, 2, rng)
    full, cells = O.propagate_full_grid(cell, filt, x, g, final_act=final_act,
                                        return_universe=True)
    roi, c = O.propagate(cell, filt, x, g, final_act=final_act, universe=True)
    np.testing.assert_allclose(c["universe"], cells, rtol=0, atol=1e-10)
    np.testing.assert_allclose(roi, full, rtol=0, atol=1e-10)
    if out is None:  # a port inside the ROI reads the same values on the port path
        port, _ = O.propagate(cell, filt, x, g, final_act=final_act)
        np.testing.assert_allclose(roi, port, rtol=0, atol=1e-10)


@pytest.mark.parametrize("final_act,bbox,pmode,out", [
    (None, None, "VALID", BORDER_PORT), ("tanh", (1, 10, 2, 10), "VALID", None),
    ("sigmoid", None, "SAME", ("rect", (0, 0), (16, 14))), ("tanh", (2, 12, 1, 9), "SAME", None)])
def test_universe_vjp_matches_finite_differences(final_act, bbox, pmode, out):
    g = O.Geometry((16, 14), (5, 3), 3, 3, [("rect", (5, 3), (4, 1)), ("rect", (4, 5), (1, 3))],
                   out or ("rect", (6, 9), (3, 1)), padding_mode=pmode)
    rng = np.random.default_rng(22)
    cell, filt = rand_cell(g, rng), rng.normal(size=(3, 1, 5, 3))
    x = rand_inputs(g, 2, rng)
    kw = dict(final_act=final_act, tau=0.7, roi_bbox=bbox, universe=True)
    out_, c = O.propagate(cell, filt, x, g, **kw)
    g_out = rng.normal(size=out_.shape)
    g_univ = rng.normal(size=c["universe"].shape)
    _, gc, gf = O.propagate_vjp(cell, filt, x, g, g_out, g_universe=g_univ, **kw)
    vc, vf = rng.normal(size=cell.shape), rng.normal(size=filt.shape)

    def L(cc, ff):
        o, k = O.propagate(cc, ff, x, g, **kw)
        return float((o * g_out).sum() + (k["universe"] * g_univ).sum())
    e = 1e-6
    fd = (L(cell + e * vc, filt + e * vf) - L(cell - e * vc, filt - e * vf)) / (2 * e)
    an = float((gc * vc).sum() + (gf * vf).sum())
    assert abs(fd - an) <= 1e-6 * max(1.0, abs(an))


@pytest.mark.parametrize("final_act,depth", [("sigmoid", 3), (None, 1)])
def test_gol_valid_full_grid_inputs_and_universe(final_act, depth):
    """VALID Game of Life (topology.py:359-388): inputs on the whole grid (the full-grid step
    0 of propagator.py:347-352) and the universe port read from the final universe equal the
    full-grid propagation; the reverse matches central finite differences."""
    n = 10
    g = O.Geometry((n, n), (3, 3), 2, depth, [("rect", (0, 0), (n, n))],
                   ("rect", (0, 0), (n, n)))
    rng = np.random.default_rng(23)
    cell, filt = rand_cell(g, rng), rng.normal(size=(2, 1, 3, 3))
    x = [rng.normal(size=(2, n, n))]
    kw = dict(final_act=final_act, universe=True)
    out, _ = O.propagate(cell, filt, x, g, **kw)
    np.testing.assert_allclose(out, O.propagate_full_grid(cell, filt, x, g, final_act=final_act),
                               rtol=0, atol=1e-10)
    g_out = rng.normal(size=out.shape)
    _, gc, gf = O.propagate_vjp(cell, filt, x, g, g_out, **kw)
    vc, vf = rng.normal(size=cell.shape), rng.normal(size=filt.shape)

    def L(cc, ff):
        return float((O.propagate(cc, ff, x, g, **kw)[0] * g_out).sum())
    e = 1e-6
    fd = (L(cell + e * vc, filt + e * vf) - L(cell - e * vc, filt - e * vf)) / (2 * e)
    an = float((gc * vc).sum() + (gf * vf).sum())
    assert abs(fd - an) <= 1e-6 * max(1.0, abs(an))


def test_zero_thresholding_gap_ste_ternary():
    """unit_milestone8_pallas_and_codd.py:239-252: replacing S by its discrete role values
    leaves the ste_ternary forward unchanged."""
    g = small_geometry(depth=3)
    rng = np.random.default_rng(12)
    cell, filt = rand_cell(g, rng), rng.normal(size=(3, 1, 5, 3))
    cell[2] = rng.uniform(-1.0, 1.2, g.grid_shape)
    x = rand_inputs(g, 2, rng)
    out, _ = O.propagate(cell, filt, x, g, mode="ste_ternary", tau=0.25)
    s = cell[2]
    roles = np.where(s >= 0.6, 2.0, s)
    roles = np.where((roles > 0) & (roles < 0.6), 1.0, roles)
    disc = cell.copy()
    disc[2] = np.where(roles >= 2.0, 1.0, np.where(roles > 0.0, 0.3, -1.0))
    out2, _ = O.propagate(disc, filt, x, g, mode="ste_ternary", tau=0.25)
    assert np.max(np.abs(out - out2)) == 0.0


# ------------------------------------------------------------------ adaptive bucketing

def _quantize_brute(lo, hi, max_len, bm):
    """The bucket by exhaustive search over every start (independent of the restatement)."""
    lo = max(0, min(lo, max_len - 1))
    hi = max(lo + 1, min(hi, max_len))
    raw = hi - lo
    if bm <= 1 or raw >= max_len:
        return 0, max_len
    q = min(max_len, -(-raw // bm) * bm)
    if q >= max_len or max_len - q < bm:
        return 0, max_len
    ideal = lo - 0.5 * (q - raw)
    valid = [s for s in range(max_len - q + 1) if s <= lo and s + q >= hi]
    for step in (max(1, bm // 2), max(1, bm // 4)):
        al = [s for s in valid if s % step == 0]
        if al:
            return min(al, key=lambda s: (abs(s - ideal), s)), min(al, key=lambda s: (
                abs(s - ideal), s)) + q
    s = max(valid[0], min(int(round(ideal)), valid[-1]))
    return s, s + q


def test_quantize_interval_exhaustive():
    for max_len in (40, 50, 17):
        for bm in (1, 4, 8, 6):
            for lo in range(0, max_len):
                for hi in range(lo + 1, max_len + 1, 3):
                    assert O.quantize_interval(lo, hi, max_len, bm) == \
                        _quantize_brute(lo, hi, max_len, bm), (lo, hi, max_len, bm)


def test_adaptive_bucket_known_answers():
    """unit_milestone7_adaptive_mask.py:52-88: the ALU chip's IO seeds give a 32x32 bucket;
    a salient bias cell at ROI (35, 44) grows it past (39, 48); 3x3 filters have radii (1,1)
    (:192-193)."""
    g = O.alu_geometry()
    rng = np.random.default_rng(13)
    cell = np.stack([rng.normal(0, 0.01, (62, 62)), np.zeros((62, 62)),
                     rng.normal(0, 0.1, (62, 62))])
    filt = rng.normal(size=(16, 1, 23, 13))
    io_roi = g.io_state_mask[11:51, 6:56]
    st, _ = O.adaptive_mask_stats(cell, filt, io_roi, g)
    r = O.quantize_interval(int(st[4]), int(st[5]), 40, 8)
    c = O.quantize_interval(int(st[6]), int(st[7]), 50, 8)
    assert (r[1] - r[0], c[1] - c[0]) == (32, 32)
    grown = cell.copy()
    grown[1, 11 + 35, 6 + 44] = 0.8
    grown[2, 11 + 35, 6 + 44] = 2.0
    st2, _ = O.adaptive_mask_stats(grown, filt, io_roi, g)
    assert st2[5] >= 39 and st2[7] >= 48
    f3 = np.zeros((4, 1, 3, 3))
    f3[:, 0] = rng.normal(size=(4, 3, 3))
    st3, _ = O.adaptive_mask_stats(cell, f3, io_roi, g)
    assert (st3[0], st3[1]) == (1, 1)


# ------------------------------------------------------------------ trainer pieces

def test_annealing_endpoints():
    """unit_milestone8_pallas_and_codd.py:274-280."""
    for sched in ("exponential", "cosine", "linear"):
        assert abs(O.annealed_temperature(0, 10, schedule=sched) - 1.0) < 1e-9
        assert abs(O.annealed_temperature(9, 10, schedule=sched) - 0.1) < 1e-9
        assert 0.1 < O.annealed_temperature(5, 10, schedule=sched) < 1.0


def test_adamw_first_step_closed_form_and_torch():
    """At step 1 the bias-corrected moments are g and g^2, so the update is
    lr*(g/(|g|+eps) + wd*p); later steps against torch.optim.AdamW (same algorithm with
    decoupled decay scaled by lr)."""
    p = RNG.normal(size=50)
    g = RNG.normal(size=50)
    p1, m, v, c = O.adamw_step(p, g, 0.0, 0.0, 0, 0.01)
    np.testing.assert_allclose(p1, p - 0.01 * (g / (np.abs(g) + 1e-8) + 1e-4 * p), rtol=1e-12)
    pt = torch.tensor(p, requires_grad=True)
    opt = torch.optim.AdamW([pt], lr=0.01, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-4)
    pp, mm, vv, cc = p, 0.0, 0.0, 0
    for k in range(4):
        gk = RNG.normal(size=50)
        pt.grad = torch.tensor(gk)
        opt.step()
        pp, mm, vv, cc = O.adamw_step(pp, gk, mm, vv, cc, 0.01)
    # torch decays before the moment update (p *= 1 - lr*wd), optax adds wd*p to the update:
    # identical to first order in lr*wd; the difference is O((lr*wd)^2) per step
    np.testing.assert_allclose(pp, pt.detach().numpy(), rtol=0, atol=1e-8)


def test_mse_gradient():
    x, y = RNG.normal(size=(4, 8, 1)), RNG.normal(size=(4, 8, 1))
    loss, g = O.mse_loss(x, y)
    assert abs(loss - float(((x - y) ** 2).mean())) < 1e-15
    xt = torch.tensor(x, requires_grad=True)
    F.mse_loss(xt, torch.tensor(y)).backward()
    np.testing.assert_allclose(g, xt.grad.numpy(), rtol=1e-12)


# ------------------------------------------------------------------ SAME / CIRCULAR modes

def mode_geometry(mode, depth=3, M=3, kernel=(5, 3), grid=(16, 16)):
    return O.Geometry(grid, kernel, M, depth, [("rect", (2, 3), (4, 1)), ("rect", (9, 5), (1, 3))],
                      ("rect", (6, 9), (3, 2)), padding_mode=mode)


def test_mode_geometry_known_answers():
    """topology.py:184-192, 256-265: VALID pads by (k-1)/2; SAME and CIRCULAR take the grid
    as ROI; CIRCULAR transforms on the grid itself."""
    v, s, c = (mode_geometry(m, kernel=(5, 3), grid=(16, 16)) for m in ("VALID", "SAME",
                                                                         "CIRCULAR"))
    assert (v.pad_h, v.pad_w, v.roi_shape, v.fft_shape) == (2, 1, (12, 14), (16, 16))
    assert (s.pad_h, s.pad_w, s.roi_shape, s.fft_shape) == (0, 0, (16, 16), (32, 32))
    assert (c.pad_h, c.pad_w, c.roi_shape, c.fft_shape) == (0, 0, (16, 16), (16, 16))


def test_circular_spectral_matches_wrap_padded_direct():
    """The grid-sized spectral correlation read modulo the grid against the reference's own
    formulation: jnp.pad(mode='wrap') then a VALID conv (brute force), and against scipy's
    'wrap' boundary correlation."""
    rng = np.random.default_rng(21)
    x, g = rng.normal(size=(2, 16, 32)), rng.normal(size=(3, 5, 7))
    pad = (2, 3)
    z_fft = O.conv2d_fft(x, g, pad, (16, 32), (16, 32))[0]
    z_dir = O.conv2d_circular_direct(x, g, pad)
    np.testing.assert_allclose(z_fft, z_dir, rtol=0, atol=1e-10)
    sc = scipy.signal.correlate2d(x[1], g[2], mode="same", boundary="wrap")
    np.testing.assert_allclose(z_dir[1, 2], sc, rtol=0, atol=1e-10)


def test_circular_adjoints():
    """<conv(x, g), gz> = <x, dx> = <g, dG> for the circular correlation, with dx and dG from
    the unshifted Plancherel backward on the grid-sized spectrum (no zero padding)."""
    rng = np.random.default_rng(22)
    x, g = rng.normal(size=(3, 16, 16)), rng.normal(size=(2, 5, 3))
    gz = rng.normal(size=(3, 2, 16, 16))
    pad = (2, 1)
    z = O.conv2d_circular_direct(x, g, pad)
    dx, dGh = O.conv2d_fft_unshifted_bwd(gz, x, g, pad, (16, 16))
    dg = O.filter_grad_from_unshifted(dGh, (5, 3), pad, (16, 16))
    lhs = float((z * gz).sum())
    assert abs(lhs - float((x * dx).sum())) <= 1e-9 * max(1.0, abs(lhs))
    assert abs(lhs - float((g * dg).sum())) <= 1e-9 * max(1.0, abs(lhs))


@pytest.mark.parametrize("mode", ["SAME", "CIRCULAR"])
def test_mode_propagate_fft_equals_direct(mode):
    g = mode_geometry(mode)
    rng = np.random.default_rng(23)
    cell, filt = rand_cell(g, rng), rng.normal(size=(3, 1, 5, 3))
    x = rand_inputs(g, 2, rng)
    a, _ = O.propagate(cell, filt, x, g)
    b, _ = O.propagate(cell, filt, x, g, conv="direct")
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-9)


@pytest.mark.parametrize("mode,final_act", [("SAME", None), ("CIRCULAR", "tanh")])
def test_mode_propagate_vjp_matches_finite_differences(mode, final_act):
    g = mode_geometry(mode)
    rng = np.random.default_rng(24)
    cell, filt = rand_cell(g, rng), rng.normal(size=(3, 1, 5, 3))
    x = rand_inputs(g, 2, rng)
    kw = dict(final_act=final_act)
    out, _ = O.propagate(cell, filt, x, g, **kw)
    g_out = rng.normal(size=out.shape)
    _, gc, gf = O.propagate_vjp(cell, filt, x, g, g_out, **kw)
    vc, vf = rng.normal(size=cell.shape), rng.normal(size=filt.shape)

    def L(c, f):
        return float((O.propagate(c, f, x, g, conv="direct", **kw)[0] * g_out).sum())
    e = 1e-6
    fd = (L(cell + e * vc, filt + e * vf) - L(cell - e * vc, filt - e * vf)) / (2 * e)
    an = float((gc * vc).sum() + (gf * vf).sum())
    assert abs(fd - an) <= 1e-6 * max(1.0, abs(an))

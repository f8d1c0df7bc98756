"""The reference-named spectral and epilogue operators of kernels_greens.py and epilogue.py
(rfft2_pruned, irfft2_pruned, conv2d_grouped_filter_grad, rfft2_filter_grad_to_oihw,
hoist_filter_rfft2, conv2d_roi_rfft_step, conv2d_valid_rfft_precomputed,
hoist_filter_rfft2_zero_fwd, conv2d_hybrid_roi_step, standardize_spatial_nchw,
fused_roi_epilogue) and inject_inputs_2d (propagator.py:103-132) on the MI355X, through the C
ABI, against float64 references: NumPy's FFTs (the JAX semantics of jnp.fft.*: an inverse real
transform keeps only the Hermitian parts of the DC and Nyquist columns), brute-force direct
correlations and their adjoints (the oracle), and torch float64 autograd on the CPU.

Bars: forward rel-L2 <= 1e-5, gradients rel-L2 <= 1e-4; exact where the reference is exact
(zero cotangents, injected values).
"""
import types

import numpy as np
import pytest
import torch

from helpers import rel_l2
from oracle import vnn_oracle as O

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-5
GRAD_TOL = 1e-4


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def _cplx(rng, shape):
    return (rng.normal(size=shape) + 1j * rng.normal(size=shape)).astype(np.complex64)


@pytest.mark.parametrize("lead,h,w,fs", [((2, 3), 20, 24, (32, 32)), ((5,), 40, 50, (64, 64)),
                                         ((2,), 30, 61, (32, 64)), ((3,), 70, 100, (128, 128))])
def test_rfft2_pruned(lead, h, w, fs):
    """kernels_greens.py:25-44 against np.fft.rfft2(s=fs); its gradient against torch
    float64 autograd of torch.fft.rfft2 for a complex cotangent."""
    from neurocell import rfft2_pruned
    rng = np.random.default_rng(50)
    x = rng.normal(size=lead + (h, w)).astype(np.float32)
    xt = dev(x).requires_grad_()
    y = rfft2_pruned(xt, fs)
    assert tuple(y.shape) == lead + (fs[0], fs[1] // 2 + 1)
    assert rel_l2(host(y), np.fft.rfft2(x.astype(np.float64), s=fs)) < FWD_TOL
    g = _cplx(rng, tuple(y.shape))
    y.backward(dev(g))
    x64 = torch.from_numpy(x).double().requires_grad_()
    torch.fft.rfft2(x64, s=fs).backward(torch.from_numpy(g).to(torch.complex128))
    assert rel_l2(host(xt.grad), x64.grad.numpy()) < GRAD_TOL


@pytest.mark.parametrize("lead,roi,pad,fs", [((2, 3), (20, 24), (3, 2), (32, 32)),
                                             ((4,), (40, 50), (11, 6), (64, 64)),
                                             ((2,), (16, 50), (10, 7), (32, 64)),
                                             ((2,), (66, 66), (31, 31), (128, 128))])
def test_irfft2_pruned(lead, roi, pad, fs):
    """kernels_greens.py:47-66 on arbitrary (non-Hermitian) complex spectra against
    np.fft.irfft2 sliced to the window; its gradient against torch float64 autograd of
    torch.fft.irfft2."""
    from neurocell import irfft2_pruned
    rng = np.random.default_rng(51)
    X = _cplx(rng, lead + (fs[0], fs[1] // 2 + 1))
    Xt = dev(X).requires_grad_()
    z = irfft2_pruned(Xt, roi, pad, fs)
    (rh, rw), (ph, pw) = roi, pad
    full = np.fft.irfft2(X.astype(np.complex128), s=fs)
    ref = full[..., ph:ph + rh, pw:pw + rw]
    assert rel_l2(host(z), ref) < FWD_TOL
    gy = rng.normal(size=tuple(z.shape)).astype(np.float32)
    z.backward(dev(gy))
    X64 = torch.from_numpy(X).to(torch.complex128).requires_grad_()
    torch.fft.irfft2(X64, s=fs)[..., ph:ph + rh, pw:pw + rw].backward(
        torch.from_numpy(gy).double())
    assert rel_l2(host(Xt.grad), X64.grad.numpy()) < GRAD_TOL


def test_rfft2_irfft2_round_trip():
    """irfft2_pruned(rfft2_pruned(x)) is x on the window at the origin (the zero padding
    removed), as jnp's pair is."""
    from neurocell import irfft2_pruned, rfft2_pruned
    x = np.random.default_rng(52).normal(size=(3, 40, 50)).astype(np.float32)
    back = irfft2_pruned(rfft2_pruned(dev(x), (64, 64)), (40, 50), (0, 0), (64, 64))
    assert rel_l2(host(back), x) < 1e-6


def _conv_case(seed, B=2, M=3, h=20, w=24, kh=7, kw=5):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(B, h, w)).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    gz = rng.normal(size=(B, M, h, w)).astype(np.float32)
    return x, g, gz, ((kh - 1) // 2, (kw - 1) // 2)


@pytest.mark.parametrize("fs", [(32, 32), (64, 64)])
def test_conv2d_roi_rfft_step_chain(fs):
    """hoist_filter_rfft2 -> conv2d_roi_rfft_step (kernels_greens.py:278-400): the SAME
    correlation and, through the shifted cotangent and the un-rolled filter gradient, the
    direct correlation's adjoints."""
    from neurocell import conv2d_roi_rfft_step, hoist_filter_rfft2
    x, g, gz, pad = _conv_case(60)
    xt, gt = dev(x).requires_grad_(), dev(g).requires_grad_()
    kf = hoist_filter_rfft2(gt, g.shape[-2:], fs)
    kf.retain_grad()
    z = conv2d_roi_rfft_step(xt, kf, x.shape[-2:], pad, fs, True)
    z.backward(dev(gz))
    with O.precision(np.float64):
        r_z = O.conv2d_direct(x, g[:, 0], pad)
        r_dx, r_dg = O.conv2d_bwd_direct(gz, x, g[:, 0], pad)
    assert rel_l2(host(z), r_z) < FWD_TOL
    assert rel_l2(host(xt.grad), r_dx) < GRAD_TOL
    assert rel_l2(host(gt.grad)[:, 0], r_dg) < GRAD_TOL
    # the ker_freq cotangent itself, kernels_greens.py:374-398: sum_b rfft2(gz zero-padded at
    # pad) * conj(rfft2(x)) in JAX's convention, whose conjugate autograd carries
    fh, fw = fs
    gpad = np.zeros(gz.shape[:2] + (fh, fw))
    gpad[:, :, pad[0]:pad[0] + gz.shape[2], pad[1]:pad[1] + gz.shape[3]] = gz
    ct = np.sum(np.fft.rfft2(gpad) * np.conj(np.fft.rfft2(x.astype(np.float64), s=fs))[:, None],
                axis=0)
    assert rel_l2(host(kf.grad), np.conj(ct)) < GRAD_TOL


def test_conv2d_roi_rfft_step_need_dx_false():
    """need_dx=False (kernels_greens.py:383-391): the cell cotangent is identically zero."""
    from neurocell import conv2d_roi_rfft_step, hoist_filter_rfft2
    x, g, gz, pad = _conv_case(61)
    xt, gt = dev(x).requires_grad_(), dev(g).requires_grad_()
    kf = hoist_filter_rfft2(gt, g.shape[-2:], (32, 32))
    conv2d_roi_rfft_step(xt, kf, x.shape[-2:], pad, (32, 32), False).backward(dev(gz))
    assert float(xt.grad.abs().max()) == 0.0
    with O.precision(np.float64):
        _, r_dg = O.conv2d_bwd_direct(gz, x, g[:, 0], pad)
    assert rel_l2(host(gt.grad)[:, 0], r_dg) < GRAD_TOL


def test_conv2d_valid_rfft_precomputed():
    """kernels_greens.py:403-425: the VALID correlation of the full grid at offset
    (Kh-1, Kw-1), and its adjoints through hoist_filter_rfft2."""
    from neurocell import conv2d_valid_rfft_precomputed, hoist_filter_rfft2
    rng = np.random.default_rng(62)
    B, M, H, W, kh, kw = 2, 3, 30, 28, 7, 5
    x = rng.normal(size=(B, H, W)).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    ho, wo = H - kh + 1, W - kw + 1
    gz = rng.normal(size=(B, M, ho, wo)).astype(np.float32)
    xt, gt = dev(x).requires_grad_(), dev(g).requires_grad_()
    kf = hoist_filter_rfft2(gt, (kh, kw), (32, 32))
    z = conv2d_valid_rfft_precomputed(xt, kf, (ho, wo), (kh, kw), (32, 32))
    z.backward(dev(gz))
    with O.precision(np.float64):
        r_z = O.conv2d_direct(x, g[:, 0], (0, 0))
        r_dx, r_dg = O.conv2d_bwd_direct(gz, x, g[:, 0], (0, 0))
    assert rel_l2(host(z), r_z) < FWD_TOL
    assert rel_l2(host(xt.grad), r_dx) < GRAD_TOL
    assert rel_l2(host(gt.grad)[:, 0], r_dg) < GRAD_TOL


def test_conv2d_hybrid_roi_step_chain():
    """hoist_filter_rfft2_zero_fwd -> conv2d_hybrid_roi_step (kernels_greens.py:428-551): the
    token is zero forward; the filters' own cotangent is zero and the token carries dG."""
    from neurocell import conv2d_hybrid_roi_step, hoist_filter_rfft2_zero_fwd
    x, g, gz, pad = _conv_case(63)
    fs = (32, 32)
    xt, gt = dev(x).requires_grad_(), dev(g).requires_grad_()
    token = hoist_filter_rfft2_zero_fwd(gt, g.shape[-2:], fs)
    assert float(token.detach().abs().max()) == 0.0
    z = conv2d_hybrid_roi_step(xt, gt, token, pad, fs, True)
    z.backward(dev(gz))
    with O.precision(np.float64):
        r_z = O.conv2d_direct(x, g[:, 0], pad)
        r_dx, r_dg = O.conv2d_bwd_direct(gz, x, g[:, 0], pad)
    assert rel_l2(host(z), r_z) < FWD_TOL
    assert rel_l2(host(xt.grad), r_dx) < GRAD_TOL
    assert rel_l2(host(gt.grad)[:, 0], r_dg) < GRAD_TOL


@pytest.mark.parametrize("B,M,h,w,hout,wout,pad", [
    (32, 3, 20, 24, 20, 24, (1, 1)),     # 3x3 SAME (the GoL / CLP filters)
    (8, 16, 24, 32, 24, 32, (11, 6)),    # 23x13 SAME on the config-4 crop
    (16, 2, 20, 24, 18, 20, (1, 1)),     # 5x7 from a smaller output window
    (4, 2, 30, 20, 24, 16, (0, 0))])     # 7x5 VALID
def test_conv2d_grouped_filter_grad(B, M, h, w, hout, wout, pad):
    """kernels_greens.py:84-123: dG of conv2d(cells, G, padding=pad) for the output cotangent,
    against the brute-force adjoint."""
    from neurocell import conv2d_grouped_filter_grad
    rng = np.random.default_rng(64)
    x = rng.normal(size=(B, h, w)).astype(np.float32)
    gz = rng.normal(size=(B, M, hout, wout)).astype(np.float32)
    kh, kw = h + 2 * pad[0] - hout + 1, w + 2 * pad[1] - wout + 1
    dg = conv2d_grouped_filter_grad(dev(x), dev(gz), pad)
    assert tuple(dg.shape) == (M, 1, kh, kw)
    with O.precision(np.float64):
        _, r_dg = O.conv2d_bwd_direct(gz, x, np.zeros((M, kh, kw)), pad)
    assert rel_l2(host(dg)[:, 0], r_dg) < GRAD_TOL


@pytest.mark.parametrize("fs,ks", [((64, 64), (23, 13)), ((32, 16), (5, 3)),
                                   ((256, 256), (31, 31))])
def test_rfft2_filter_grad_to_oihw(fs, ks):
    """kernels_greens.py:262-275 on an arbitrary complex cotangent: flip(irfft2(.)[:Kh, :Kw])
    with NumPy's inverse."""
    from neurocell import rfft2_filter_grad_to_oihw
    G = _cplx(np.random.default_rng(65), (4, fs[0], fs[1] // 2 + 1))
    out = rfft2_filter_grad_to_oihw(dev(G), ks, fs)
    ref = np.flip(np.fft.irfft2(G.astype(np.complex128), s=fs)[:, :ks[0], :ks[1]], (-2, -1))
    assert rel_l2(host(out)[:, 0], ref) < FWD_TOL


def test_hoist_filter_rfft2_pairing():
    """hoist_filter_rfft2 (kernels_greens.py:278-313): forward = rfft2 of the flipped filters;
    its backward is rfft2_filter_grad_to_oihw of the JAX-convention cotangent (the conjugate
    of autograd's)."""
    from neurocell import hoist_filter_rfft2
    rng = np.random.default_rng(66)
    g = rng.normal(size=(3, 1, 9, 7)).astype(np.float32)
    gt = dev(g).requires_grad_()
    kf = hoist_filter_rfft2(gt, (9, 7), (32, 32))
    ref = np.fft.rfft2(np.flip(g[:, 0].astype(np.float64), (-2, -1)), s=(32, 32))
    assert rel_l2(host(kf), ref) < FWD_TOL
    G = _cplx(rng, tuple(kf.shape))
    kf.backward(dev(G))
    r = np.flip(np.fft.irfft2(np.conj(G).astype(np.complex128), s=(32, 32))[:, :9, :7], (-2, -1))
    assert rel_l2(host(gt.grad)[:, 0], r) < GRAD_TOL


@pytest.mark.parametrize("shape", [(3, 4, 40, 50), (2, 2, 96, 100), (5, 7, 3)])
def test_standardize_spatial_nchw(shape):
    """epilogue.py:20-25: per-plane standardisation (population variance, eps 1e-5) and its
    gradient against torch float64 autograd."""
    from neurocell import standardize_spatial_nchw
    rng = np.random.default_rng(67)
    z = (rng.normal(size=shape) * 3 + 1).astype(np.float32)
    zt = dev(z).requires_grad_()
    out = standardize_spatial_nchw(zt)
    z64 = torch.from_numpy(z).double().requires_grad_()
    mu = z64.mean(dim=(-2, -1), keepdim=True)
    ref = (z64 - mu) / torch.sqrt(((z64 - mu) ** 2).mean(dim=(-2, -1), keepdim=True) + 1e-5)
    assert rel_l2(host(out), ref.detach().numpy()) < FWD_TOL
    g = rng.normal(size=shape).astype(np.float32)
    out.backward(dev(g))
    ref.backward(torch.from_numpy(g).double())
    assert rel_l2(host(zt.grad), z64.grad.numpy()) < GRAD_TOL


def test_fused_roi_epilogue():
    """epilogue.py:59-79: the ROI update embedded into the full-grid border template; the
    template's ROI cells get no gradient, its border cells the cotangent itself."""
    from neurocell import fused_roi_epilogue
    from neurocell.topology import ChipTopology2D
    topo = ChipTopology2D.alu_chip(out_width=2)
    H, W = topo.grid_shape
    h, w = topo.roi_shape
    rng = np.random.default_rng(68)
    B, M = 3, 16
    z = rng.normal(size=(B, M, h, w)).astype(np.float32)
    wv, sv, bv = (rng.normal(size=(h, w)).astype(np.float32) for _ in range(3))
    cb = rng.normal(size=(B, H, W)).astype(np.float32)
    zt, cbt = dev(z).requires_grad_(), dev(cb).requires_grad_()
    sp = types.SimpleNamespace(w_eff_roi=dev(wv), s_eff_roi=dev(sv), b_roi=dev(bv))
    out = fused_roi_epilogue(zt, sp, cbt, topo, "tanh")
    r_roi, mean, rstd = O.epilogue_fwd(z, np.zeros((M, h, w)), wv, sv, bv, "tanh", False)
    ref = cb.astype(np.float64).copy()
    rh, rw = topo.pad_h, topo.pad_w
    ref[:, rh:H - rh, rw:W - rw] = r_roi
    assert rel_l2(host(out), ref) < FWD_TOL
    g = rng.normal(size=(B, H, W)).astype(np.float32)
    out.backward(dev(g))
    r = O.epilogue_bwd(z, np.zeros((M, h, w)), wv, sv, bv, mean, rstd,
                       g[:, rh:H - rh, rw:W - rw], "tanh", False)
    assert rel_l2(host(zt.grad), r[0]) < GRAD_TOL
    gcb = g.copy()
    gcb[:, rh:H - rh, rw:W - rw] = 0.0
    assert np.array_equal(host(cbt.grad), gcb)


@pytest.mark.parametrize("chip", ["alu", "clp", "gol"])
def test_inject_inputs_2d(chip):
    """propagator.py:103-132: the port inputs written into a zero (B, H, W) grid, exactly;
    the ALU's ctrl operand as an 8x1 column (its per-port input is (B, 8, 1) although the
    port is declared 1x8)."""
    from neurocell import inject_inputs_2d
    from neurocell.topology import ChipTopology2D
    rng = np.random.default_rng(69)
    if chip == "alu":
        topo = ChipTopology2D.alu_chip(out_width=2)
        geom = O.alu_geometry(out_width=2)
        x = rng.normal(size=(4, 3, 8, 1)).astype(np.float32)
    elif chip == "clp":
        topo = ChipTopology2D.clp_chip(n=8)
        geom = O.Geometry((8, 8), (3, 3), 1, 4, [("coords", list(topo.in_ports[0].coords))],
                          ("coords", list(topo.out_port.coords)))
        x = rng.normal(size=(4, 2)).astype(np.float32)
    else:
        topo = ChipTopology2D.gol_chip(n=16, kernel_size=(3, 3), directions=4, depth=2)
        geom = O.Geometry((16, 16), (3, 3), 4, 2, [("rect", (0, 0), (16, 16))],
                          ("rect", (0, 0), (16, 16)))
        x = rng.normal(size=(4, 16, 16)).astype(np.float32)
    cells = inject_inputs_2d(dev(x), topo)
    ref = O.inject_inputs_full(O.split_ports(x, geom), geom)
    assert np.array_equal(host(cells), ref.astype(np.float32))

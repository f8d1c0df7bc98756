"""Entry-point parity cases for the C ABI, run on two backends:

* ``HostBackend``: NumPy host buffers against the CPU-emulated build of the kernel sources
  (``tests/emu``) - checks the kernels' indexing and arithmetic without a GPU;
* ``DeviceBackend``: torch device tensors against the gfx950 library on the MI355X.

Every case compares the entry point with the float64 oracle on the same seeded inputs and
returns {name: rel-L2 error}; the bars are fp32-level (see ``TOL``).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from oracle import vnn_oracle as O
from helpers import rel_l2
from neurocell import _abi

TOL = 2e-6  # fp32 arithmetic against the float64 oracle, per entry point


class HostBackend:
    def __init__(self, lib):
        self.lib = lib

    def put(self, a, dtype=np.float32):
        return np.ascontiguousarray(np.asarray(a), dtype=dtype)

    def zeros(self, shape, dtype=np.float32):
        return np.zeros(shape, dtype)

    def ptr(self, t):
        return None if t is None else t.ctypes.data_as(C.c_void_p)

    def get(self, t):
        return np.asarray(t)

    def stream(self):
        return None

    def sync(self):
        pass


class DeviceBackend:
    def __init__(self, lib):
        import torch
        self.lib = lib
        self.torch = torch
        self.dev = torch.device("cuda")

    def put(self, a, dtype=np.float32):
        return self.torch.from_numpy(np.ascontiguousarray(np.asarray(a), dtype=dtype)).to(self.dev)

    def zeros(self, shape, dtype=np.float32):
        t = {np.float32: self.torch.float32, np.int32: self.torch.int32,
             np.uint8: self.torch.uint8}[dtype]
        return self.torch.zeros(shape, dtype=t, device=self.dev)

    def ptr(self, t):
        return None if t is None else C.c_void_p(t.data_ptr())

    def get(self, t):
        self.torch.cuda.synchronize()
        return t.cpu().numpy()

    def stream(self):
        return C.c_void_p(self.torch.cuda.current_stream().cuda_stream)

    def sync(self):
        self.torch.cuda.synchronize()


def _ok(be, status, what):
    _abi.check(be.lib, status, what)


def _cplx(a):
    a = np.asarray(a)
    return a[..., 0] + 1j * a[..., 1]


def case_fftconv(be, B=3, M=5, hin=10, win=12, kh=5, kw=3, FH=16, FW=16, seed=0):
    """Spectral correlation forward/backward and the filter spectrum, SAME-ROI shift."""
    rng = np.random.default_rng(seed)
    ph, pw = (kh - 1) // 2, (kw - 1) // 2
    x = rng.normal(size=(B, hin, win)).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    gz = rng.normal(size=(B, M, hin, win)).astype(np.float32)
    L, s = be.lib, be.stream()
    xd, gd = be.put(x), be.put(g)
    ghat = be.zeros((M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_filter_spectrum_fwd(s, M, kh, kw, FH, FW, be.ptr(gd), be.ptr(ghat)), "spec")
    z = be.zeros((B, M, hin, win))
    xhat = be.zeros((B, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_fftconv_fwd(s, B, M, hin, win, hin, win, ph, pw, FH, FW, be.ptr(xd),
                             be.ptr(ghat), be.ptr(z), be.ptr(xhat)), "fwd")
    ws = be.zeros((L.nc_fftconv_bwd_workspace_size(B, M, FH, FW) // 4 + 1,))
    dx = be.zeros((B, hin, win))
    dgh = be.zeros((M, FH, FW // 2 + 1, 2))
    gzd = be.put(gz)
    # the batch-summed cotangent spectra: written by the first call, added to by the second
    ssum = be.zeros((M, FH, FW // 2 + 1, 2))
    nb = ws.nbytes if hasattr(ws, "nbytes") else ws.numel() * 4
    for acc in (0, 1):
        _ok(be, L.nc_fftconv_bwd_ex(s, B, M, hin, win, hin, win, ph, pw, FH, FW, be.ptr(gzd),
                                    be.ptr(xhat), be.ptr(ghat), 1, be.ptr(dx), be.ptr(dgh), 0, 0,
                                    be.ptr(ssum), acc, be.ptr(ws), nb), "bwd")
    gf = be.zeros((M, 1, kh, kw))
    _ok(be, L.nc_filter_spectrum_bwd(s, M, kh, kw, FH, FW, ph, pw, be.ptr(dgh), be.ptr(gf), 0,
                                     0), "specbwd")
    # the row-stack variant: two accumulating calls, summed by the consumers
    npart = L.nc_fftconv_bwd_partials(B, M, FH, FW)
    dgp = be.zeros((npart, M, FH, FW // 2 + 1, 2))
    sp = be.zeros((npart, M, FH, FW // 2 + 1, 2))
    for acc in (0, 1):
        _ok(be, L.nc_fftconv_bwd_parts(s, B, M, hin, win, hin, win, ph, pw, FH, FW, be.ptr(gzd),
                                       be.ptr(xhat), be.ptr(ghat), 0, None, be.ptr(dgp), acc, 0,
                                       be.ptr(sp), acc, be.ptr(ws), nb), "bwd_parts")
    dgs = be.zeros((M, FH, FW // 2 + 1, 2))
    ssm = be.zeros((M, FH, FW // 2 + 1, 2))
    n2 = M * FH * (FW // 2 + 1) * 2
    jobs = _abi.rows_jobs((be.ptr(dgp).value, be.ptr(dgs).value, n2, 0, npart),
                          (be.ptr(sp).value, be.ptr(ssm).value, n2, 0, npart))
    _ok(be, L.nc_rows_sum(s, 2, jobs), "rows_sum")
    gf2 = be.zeros((M, 1, kh, kw))
    _ok(be, L.nc_filter_spectrum_bwd(s, M, kh, kw, FH, FW, ph, pw, be.ptr(dgs), be.ptr(gf2), 0,
                                     0), "specbwd_rows")
    dxr, dgr = O.conv2d_bwd_direct(gz, x, g[:, 0], (ph, pw))
    return {
        "dG_parts": rel_l2(be.get(gf2)[:, 0], 2 * dgr),
        "gz_hat_sum_parts": rel_l2(_cplx(be.get(ssm)),
                                   2 * np.fft.rfft2(gz.astype(np.float64).sum(0), s=(FH, FW))),
        "ghat": rel_l2(_cplx(be.get(ghat)), O.filter_spectrum(g[:, 0], (FH, FW))),
        "xhat": rel_l2(_cplx(be.get(xhat)), np.fft.rfft2(x.astype(np.float64), s=(FH, FW))),
        "z": rel_l2(be.get(z), O.conv2d_direct(x, g[:, 0], (ph, pw))),
        "dx": rel_l2(be.get(dx), dxr),
        "dG": rel_l2(be.get(gf)[:, 0], dgr),
        "dghat": rel_l2(_cplx(be.get(dgh)),
                        O.conv2d_fft_unshifted_bwd(gz, x, g[:, 0], (ph, pw), (FH, FW))[1]),
        # linearity: sum_b rfft2(gz_b) = rfft2(sum_b gz_b), twice (the accumulate call)
        "gz_hat_sum": rel_l2(_cplx(be.get(ssum)),
                             2 * np.fft.rfft2(gz.astype(np.float64).sum(0), s=(FH, FW))),
    }


def case_border_conv(be, M=4, h=12, w=10, kh=7, kw=5, FH=32, FW=16, seed=1):
    """VALID correlation of a (h+kh-1, w+kw-1) patch: the hoisted border conv and its reverse."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    Hp, Wp = h + kh - 1, w + kw - 1
    patch = rng.normal(size=(1, Hp, Wp)).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    gd = be.put(g)
    ghat = be.zeros((M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_filter_spectrum_fwd(s, M, kh, kw, FH, FW, be.ptr(gd), be.ptr(ghat)), "spec")
    dl = be.zeros((1, M, h, w))
    phat = be.zeros((1, FH, FW // 2 + 1, 2))
    pd = be.put(patch)
    _ok(be, L.nc_fftconv_fwd(s, 1, M, Hp, Wp, h, w, kh - 1, kw - 1, FH, FW, be.ptr(pd),
                             be.ptr(ghat), be.ptr(dl), be.ptr(phat)), "fwd")
    gdl = rng.normal(size=(1, M, h, w)).astype(np.float32)
    gdd = be.put(gdl)
    gp = be.zeros((1, Hp, Wp))
    dgh = be.zeros((M, FH, FW // 2 + 1, 2))
    ws = be.zeros((L.nc_fftconv_bwd_workspace_size(1, M, FH, FW) // 4 + 1,))
    nb = ws.nbytes if hasattr(ws, "nbytes") else ws.numel() * 4
    _ok(be, L.nc_fftconv_bwd(s, 1, M, Hp, Wp, h, w, kh - 1, kw - 1, FH, FW, be.ptr(gdd),
                             be.ptr(phat), be.ptr(ghat), 1, be.ptr(gp), be.ptr(dgh), 0, 0,
                             be.ptr(ws), nb), "bwd")
    gf = be.zeros((M, 1, kh, kw))
    _ok(be, L.nc_filter_spectrum_bwd(s, M, kh, kw, FH, FW, kh - 1, kw - 1, be.ptr(dgh),
                                     be.ptr(gf), 0, 0), "specbwd")
    gpr, ggr = O.conv2d_bwd_direct(gdl, patch, g[:, 0], (0, 0))
    # the same reverse from the cotangent's spectra (nc_fftconv_bwd_hat), the spectra taken
    # as the batch sum of a two-sample cotangent whose samples add up to gdl
    half = rng.normal(size=(1, M, h, w)).astype(np.float32)
    g2 = be.put(np.concatenate([half, gdl - half]))
    ws2 = be.zeros((L.nc_fftconv_bwd_workspace_size(2, M, FH, FW) // 4 + 1,))
    nb2 = ws2.nbytes if hasattr(ws2, "nbytes") else ws2.numel() * 4
    x2 = be.zeros((2, FH, FW // 2 + 1, 2))
    dgx = be.zeros((M, FH, FW // 2 + 1, 2))
    ssum = be.zeros((M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_fftconv_bwd_ex(s, 2, M, Hp, Wp, h, w, kh - 1, kw - 1, FH, FW, be.ptr(g2),
                                be.ptr(x2), be.ptr(ghat), 0, None, be.ptr(dgx), 0, 0,
                                be.ptr(ssum), 0, be.ptr(ws2), nb2), "bwd_ex")
    gp2 = be.zeros((1, Hp, Wp))
    dgh2 = be.zeros((M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_fftconv_bwd_hat(s, M, Hp, Wp, kh - 1, kw - 1, FH, FW, be.ptr(ssum),
                                 be.ptr(phat), be.ptr(ghat), be.ptr(gp2), be.ptr(dgh2), 0, 0,
                                 be.ptr(ws), nb), "bwd_hat")
    # the same from row stacks (nc_fftconv_bwd_parts -> nc_fftconv_bwd_hat_parts)
    npart = L.nc_fftconv_bwd_partials(2, M, FH, FW)
    sp = be.zeros((npart, M, FH, FW // 2 + 1, 2))
    dgxp = be.zeros((npart, M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_fftconv_bwd_parts(s, 2, M, Hp, Wp, h, w, kh - 1, kw - 1, FH, FW, be.ptr(g2),
                                   be.ptr(x2), be.ptr(ghat), 0, None, be.ptr(dgxp), 0, 0,
                                   be.ptr(sp), 0, be.ptr(ws2), nb2), "bwd_parts")
    ssm = be.zeros((M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_rows_sum(s, 1, _abi.rows_jobs((be.ptr(sp).value, be.ptr(ssm).value,
                                                M * FH * (FW // 2 + 1) * 2, 0, npart))),
        "rows_sum")
    gp3 = be.zeros((1, Hp, Wp))
    _ok(be, L.nc_fftconv_bwd_hat(s, M, Hp, Wp, kh - 1, kw - 1, FH, FW, be.ptr(ssm), None,
                                 be.ptr(ghat), be.ptr(gp3), None, 0, 0, be.ptr(ws), nb),
        "bwd_hat_rows")
    gf2 = be.zeros((M, 1, kh, kw))
    _ok(be, L.nc_filter_spectrum_bwd(s, M, kh, kw, FH, FW, kh - 1, kw - 1, be.ptr(dgh2),
                                     be.ptr(gf2), 0, 0), "specbwd2")
    return {"delta": rel_l2(be.get(dl), O.conv2d_direct(patch, g[:, 0], (0, 0))),
            "dpatch": rel_l2(be.get(gp), gpr), "dG": rel_l2(be.get(gf)[:, 0], ggr),
            "dpatch_hat": rel_l2(be.get(gp2), gpr), "dG_hat": rel_l2(be.get(gf2)[:, 0], ggr),
            "dpatch_hat_parts": rel_l2(be.get(gp3), gpr)}


def case_border_fold(be, B=3, M=4, h=12, w=10, kh=7, kw=5, FH=32, FW=16, seed=5):
    """The border conv folded into a SAME-ROI correlation: xhat_add = the patch spectrum
    shifted onto the ROI window (nc_plane_spectrum), its reverse through nc_fftconv_bwd_ex
    (dG of both terms, the cotangent spectrum sum) and nc_fftconv_bwd_hat (patch gradient)."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    ph, pw = (kh - 1) // 2, (kw - 1) // 2
    Hp, Wp = h + kh - 1, w + kw - 1
    sh, sw = (ph - (kh - 1)) % FH, (pw - (kw - 1)) % FW
    x = rng.normal(size=(B, h, w)).astype(np.float32)
    patch = rng.normal(size=(1, Hp, Wp)).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    gz = rng.normal(size=(B, M, h, w)).astype(np.float32)
    # operands held in names: a device tensor must outlive the launch that reads it
    gd, patchd, xd, gzd = be.put(g), be.put(patch), be.put(x), be.put(gz)
    ghat = be.zeros((M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_filter_spectrum_fwd(s, M, kh, kw, FH, FW, be.ptr(gd), be.ptr(ghat)), "spec")
    padd = be.zeros((1, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_plane_spectrum(s, 1, Hp, Wp, FH, FW, sh, sw, be.ptr(patchd),
                                be.ptr(padd)), "plane_spectrum")
    z = be.zeros((B, M, h, w))
    xhat = be.zeros((B, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_fftconv_fwd_ex(s, B, M, h, w, h, w, ph, pw, FH, FW, be.ptr(xd),
                                be.ptr(padd), be.ptr(ghat), be.ptr(z), be.ptr(xhat)), "fwd_ex")
    ws = be.zeros((L.nc_fftconv_bwd_workspace_size(B, M, FH, FW) // 4 + 1,))
    nb = ws.nbytes if hasattr(ws, "nbytes") else ws.numel() * 4
    dx = be.zeros((B, h, w))
    dgh = be.zeros((M, FH, FW // 2 + 1, 2))
    ssum = be.zeros((M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_fftconv_bwd_ex(s, B, M, h, w, h, w, ph, pw, FH, FW, be.ptr(gzd),
                                be.ptr(xhat), be.ptr(ghat), 1, be.ptr(dx), be.ptr(dgh), 0, 0,
                                be.ptr(ssum), 0, be.ptr(ws), nb), "bwd_ex")
    gf = be.zeros((M, 1, kh, kw))
    _ok(be, L.nc_filter_spectrum_bwd(s, M, kh, kw, FH, FW, ph, pw, be.ptr(dgh), be.ptr(gf), 0,
                                     0), "specbwd")
    gp = be.zeros((1, Hp, Wp))
    _ok(be, L.nc_fftconv_bwd_hat(s, M, Hp, Wp, kh - 1, kw - 1, FH, FW, be.ptr(ssum), None,
                                 be.ptr(ghat), be.ptr(gp), None, 0, 0, be.ptr(ws), nb), "bwd_hat")
    # both in one launch
    gf2, gp2 = be.zeros((M, 1, kh, kw)), be.zeros((1, Hp, Wp))
    _ok(be, L.nc_filter_patch_bwd(s, M, kh, kw, FH, FW, ph, pw, be.ptr(dgh), be.ptr(gf2), 0, 0,
                                  Hp, Wp, kh - 1, kw - 1, be.ptr(ssum), be.ptr(ghat),
                                  be.ptr(gp2), be.ptr(ws), nb), "filter_patch")
    # references: the shifted spectrum from NumPy's rfft2 of the rolled plane; the rest from
    # brute-force correlations of the two terms
    grid = np.zeros((FH, FW))
    grid[:Hp, :Wp] = patch[0]
    shifted = np.fft.rfft2(np.roll(grid, (sh, sw), axis=(0, 1)))
    gk = g[:, 0]
    delta = O.conv2d_direct(patch, gk, (0, 0))                       # (1, M, h, w)
    dxr, dgr = O.conv2d_bwd_direct(gz, x, gk, (ph, pw))
    gpr, dgb = O.conv2d_bwd_direct(gz.astype(np.float64).sum(0, keepdims=True), patch, gk, (0, 0))
    return {"shifted_spectrum": rel_l2(_cplx(be.get(padd))[0], shifted),
            "z": rel_l2(be.get(z), O.conv2d_direct(x, gk, (ph, pw)) + delta),
            "dx": rel_l2(be.get(dx), dxr), "dG": rel_l2(be.get(gf)[:, 0], dgr + dgb),
            "dpatch": rel_l2(be.get(gp), gpr),
            "dG_one_launch": rel_l2(be.get(gf2)[:, 0], dgr + dgb),
            "dpatch_one_launch": rel_l2(be.get(gp2), gpr)}


def case_plane_spectra(be, B=3, M=4, h=12, w=10, kh=7, kw=5, FH=32, FW=16, seed=6):
    """nc_plane_spectra with all four job kinds in one call (filter spectra, a shifted plane, a
    plain and an added-to cell spectrum) and nc_spectral_correlate on its outputs."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    ph, pw = (kh - 1) // 2, (kw - 1) // 2
    Hp, Wp = h + kh - 1, w + kw - 1
    sh, sw = 3 % FH, (FW - 2) % FW
    x = rng.normal(size=(B, h, w)).astype(np.float32)
    patch = rng.normal(size=(1, Hp, Wp)).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    A = (rng.normal(size=(FH, FW // 2 + 1)) + 1j * rng.normal(size=(FH, FW // 2 + 1)))
    Ad = be.put(np.stack([A.real, A.imag], -1))
    xd, pd, gd = be.put(x), be.put(patch), be.put(g)
    ghat = be.zeros((M, FH, FW // 2 + 1, 2))
    phat = be.zeros((1, FH, FW // 2 + 1, 2))
    xhat = be.zeros((B, FH, FW // 2 + 1, 2))
    xhat2 = be.zeros((B, FH, FW // 2 + 1, 2))
    a = lambda t: be.ptr(t).value
    jobs = _abi.spectrum_jobs((a(gd), a(ghat), None, M, kh, kw, 1, 0, 0),
                              (a(pd), a(phat), None, 1, Hp, Wp, 0, sh, sw),
                              (a(xd), a(xhat), None, B, h, w, 0, 0, 0),
                              (a(xd), a(xhat2), a(Ad), B, h, w, 0, 0, 0))
    _ok(be, L.nc_plane_spectra(s, FH, FW, 4, jobs), "plane_spectra")
    z = be.zeros((B, M, h, w))
    _ok(be, L.nc_spectral_correlate(s, B, M, h, w, ph, pw, FH, FW, be.ptr(xhat), be.ptr(ghat),
                                    be.ptr(z)), "correlate")
    grid = np.zeros((FH, FW))
    grid[:Hp, :Wp] = patch[0]
    xs = np.fft.rfft2(x.astype(np.float64), s=(FH, FW))
    return {"ghat": rel_l2(_cplx(be.get(ghat)), O.filter_spectrum(g[:, 0], (FH, FW))),
            "shifted": rel_l2(_cplx(be.get(phat))[0],
                              np.fft.rfft2(np.roll(grid, (sh, sw), axis=(0, 1)))),
            "xhat": rel_l2(_cplx(be.get(xhat)), xs),
            "xhat_add": rel_l2(_cplx(be.get(xhat2)), xs + A[None]),
            "z": rel_l2(be.get(z), O.conv2d_direct(x, g[:, 0], (ph, pw)))}


def case_epilogue_fftconv_bwd(be, B=2, M=3, h=112, w=112, kh=31, kw=21, FH=256, FW=256,
                              act="tanh", seed=12):
    """One hidden layer's reverse step through nc_epilogue_fftconv_bwd_parts against its two
    entries run in turn (nc_epilogue_bwd_parts writing gz, nc_fftconv_bwd_parts reading it):
    max |difference| / max |value| of dx, the dghat and gz_hat_sum rows and the gw/gs/gb rows
    (0 where gz's values are formed by the same arithmetic), plus the fused path's dx against
    the oracle's correlation backward of the oracle epilogue's gz."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    ph, pw = (kh - 1) // 2, (kw - 1) // 2
    N = h * w
    x = rng.normal(size=(B, h, w)).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    xd, gd = be.put(x), be.put(g)
    ghat = be.zeros((M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_filter_spectrum_fwd(s, M, kh, kw, FH, FW, be.ptr(gd), be.ptr(ghat)), "spec")
    zd, xhat = be.zeros((B, M, h, w)), be.zeros((B, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_fftconv_fwd(s, B, M, h, w, h, w, ph, pw, FH, FW, be.ptr(xd), be.ptr(ghat),
                             be.ptr(zd), be.ptr(xhat)), "fwd")
    wv = rng.normal(size=(h, w)).astype(np.float32)
    sv = rng.uniform(size=(h, w)).astype(np.float32)
    bv = rng.normal(size=(h, w)).astype(np.float32)
    gy = rng.normal(size=(B, h, w)).astype(np.float32)
    wd, sd, bd, gyd = (be.put(a) for a in (wv, sv, bv, gy))
    aid = _abi.ACT_IDS[act]
    n_epi = L.nc_epilogue_workspace_size(B, M, h, w)
    ws_e = be.zeros((n_epi // 4 + 1,))
    out, mean, rstd = be.zeros((B, h, w)), be.zeros((B, M)), be.zeros((B, M))
    _ok(be, L.nc_epilogue_fwd(s, B, M, h, w, aid, 0.01, 0, be.ptr(zd), None, be.ptr(wd),
                              be.ptr(sd), be.ptr(bd), be.ptr(out), be.ptr(mean), be.ptr(rstd),
                              be.ptr(ws_e), n_epi), "epi")
    n_fc = L.nc_fftconv_bwd_workspace_size(B, M, FH, FW)
    ws_f = be.zeros((n_fc // 4 + 1,))
    R, npart = L.nc_epilogue_bwd_partials(B, M, h, w), L.nc_fftconv_bwd_partials(B, M, FH, FW)
    spec = (npart, M, FH, FW // 2 + 1, 2)
    res = {}
    outs = []
    for fused in (False, True):
        pg, dx = be.zeros((3, R * N)), be.zeros((B, h, w))
        dg, ss = be.zeros(spec), be.zeros(spec)
        gz = be.zeros((B, M, h, w))
        if fused:
            _ok(be, L.nc_epilogue_fftconv_bwd_parts(
                s, B, M, h, w, aid, 0.01, be.ptr(zd), be.ptr(wd), be.ptr(sd), be.ptr(bd),
                be.ptr(mean), be.ptr(rstd), be.ptr(gyd), be.ptr(gz), be.ptr(pg), R * N, h, w,
                ph, pw, FH, FW, be.ptr(xhat), be.ptr(ghat), 1, be.ptr(dx), be.ptr(dg), 0, 0,
                be.ptr(ss), 0, be.ptr(ws_e), n_epi, be.ptr(ws_f), n_fc), "fused")
        else:
            _ok(be, L.nc_epilogue_bwd_parts(s, B, M, h, w, aid, 0.01, 0, be.ptr(zd), None,
                                            be.ptr(wd), be.ptr(sd), be.ptr(bd), be.ptr(mean),
                                            be.ptr(rstd), be.ptr(gyd), be.ptr(gz), be.ptr(pg),
                                            R * N, be.ptr(ws_e), n_epi), "epib_parts")
            _ok(be, L.nc_fftconv_bwd_parts(s, B, M, h, w, h, w, ph, pw, FH, FW, be.ptr(gz),
                                           be.ptr(xhat), be.ptr(ghat), 1, be.ptr(dx),
                                           be.ptr(dg), 0, 0, be.ptr(ss), 0, be.ptr(ws_f), n_fc),
                "bwd_parts")
            gz_sep = be.get(gz)
        outs.append([be.get(a) for a in (dx, dg, ss, pg)])
    for name, a, b in zip(("dx", "dghat_rows", "gz_hat_sum_rows", "pg_rows"), *outs):
        res[name] = float(np.abs(b - a).max() / max(np.abs(a).max(), 1e-30))
    # the oracle's gz (its epilogue backward on the same z) through the oracle correlation
    gz_r = O.epilogue_bwd(be.get(zd), np.zeros((M, h, w), np.float32), wv, sv, bv,
                          be.get(mean), be.get(rstd), gy, act, False)[0]
    dxr, _ = O.conv2d_bwd_direct(gz_r, x, g[:, 0], (ph, pw))
    res["dx_vs_oracle"] = rel_l2(outs[1][0], dxr)
    res["gz_vs_oracle"] = rel_l2(gz_sep, gz_r)
    return res


def case_epilogue(be, B=3, M=5, h=10, w=12, act="tanh", has_border=1, seed=2):
    """Hidden-step epilogue forward/backward (single-pass N <= 8192, tiled above)."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    z = (rng.normal(size=(B, M, h, w)) * 2 + 0.5).astype(np.float32)
    d = rng.normal(size=(M, h, w)).astype(np.float32)
    wv = rng.normal(size=(h, w)).astype(np.float32)
    sv = rng.uniform(size=(h, w)).astype(np.float32)
    bv = rng.normal(size=(h, w)).astype(np.float32)
    gy = rng.normal(size=(B, h, w)).astype(np.float32)
    zd, dd, wd, sd, bd, gyd = (be.put(a) for a in (z, d, wv, sv, bv, gy))
    out, mean, rstd = be.zeros((B, h, w)), be.zeros((B, M)), be.zeros((B, M))
    ws = be.zeros((L.nc_epilogue_workspace_size(B, M, h, w) // 4 + 1,))
    nb = ws.nbytes if hasattr(ws, "nbytes") else ws.numel() * 4
    aid = _abi.ACT_IDS[act]
    _ok(be, L.nc_epilogue_fwd(s, B, M, h, w, aid, 0.01, has_border, be.ptr(zd), be.ptr(dd),
                              be.ptr(wd), be.ptr(sd), be.ptr(bd), be.ptr(out), be.ptr(mean),
                              be.ptr(rstd), be.ptr(ws), nb), "epi")
    # gdb starts non-zero: without the border term the entry point writes exact zeros
    # (the reference's zeros_like cotangent, unit_milestone6_general_vnn.py:107-110)
    gz, gdb = be.zeros((B, M, h, w)), be.put(np.full((M, h, w), 7.0, np.float32))
    gw, gs, gb = be.zeros((h, w)), be.zeros((h, w)), be.zeros((h, w))
    _ok(be, L.nc_epilogue_bwd(s, B, M, h, w, aid, 0.01, has_border, be.ptr(zd), be.ptr(dd),
                              be.ptr(wd), be.ptr(sd), be.ptr(bd), be.ptr(mean), be.ptr(rstd),
                              be.ptr(gyd), be.ptr(gz), be.ptr(gdb), be.ptr(gw), be.ptr(gs),
                              be.ptr(gb), 0, 0, be.ptr(ws), nb), "epib")
    o_r, m_r, r_r = O.epilogue_fwd(z, d, wv, sv, bv, act, bool(has_border))
    r = O.epilogue_bwd(z, d, wv, sv, bv, m_r, r_r, gy, act, bool(has_border))
    res = {"out": rel_l2(be.get(out), o_r), "mean": rel_l2(be.get(mean), m_r),
           "rstd": rel_l2(be.get(rstd), r_r)}
    # the row-stack variant, written as the second of two steps' row blocks (padded plane
    # stride) and summed by nc_rows_sum: the same reduction over the same rows, bit for bit
    R = L.nc_epilogue_bwd_partials(B, M, h, w)
    N = h * w
    stride = 2 * R * N + 5
    pg = be.zeros((3 * stride,))
    gz2, gsum = be.zeros((B, M, h, w)), be.zeros((3, N))
    a = lambda t, off=0: be.ptr(t).value + 4 * off
    _ok(be, L.nc_epilogue_bwd_parts(s, B, M, h, w, aid, 0.01, has_border, be.ptr(zd), be.ptr(dd),
                                    be.ptr(wd), be.ptr(sd), be.ptr(bd), be.ptr(mean),
                                    be.ptr(rstd), be.ptr(gyd), be.ptr(gz2), a(pg, R * N), stride,
                                    be.ptr(ws), nb), "epib_parts")
    jobs = _abi.rows_jobs(*[(a(pg, i * stride + R * N), a(gsum, i * N), N, 0, R)
                            for i in range(3)])
    _ok(be, L.nc_rows_sum(s, 3, jobs), "rows_sum")
    gsum = be.get(gsum)
    res["parts_gz_mismatch"] = float((be.get(gz2) != be.get(gz)).sum())
    res["parts_params_mismatch"] = float(sum((gsum[i] != be.get(t).reshape(-1)).sum()
                                             for i, t in enumerate((gw, gs, gb))))
    for k, a, b in zip(("gz", "gdb", "gw", "gs", "gb"), (gz, gdb, gw, gs, gb), r):
        if k == "gdb" and not has_border:
            res["gdb_nonzero"] = float((be.get(gdb) != 0.0).sum())
            continue
        res[k] = rel_l2(be.get(a), b)
    return res


def case_epilogue_parts(be, B=3, M=9, h=10, w=12, kh=5, kw=3, FH=16, FW=16, seed=7):
    """nc_epilogue_fwd_parts + nc_fftconv_fwd_parts against nc_epilogue_fwd + nc_fftconv_fwd:
    the partial planes add up to the combined output and the correlation from them matches,
    both bit for bit (the same fixed-order sums), and the output matches the oracle."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    z = (rng.normal(size=(B, M, h, w)) * 2 + 0.5).astype(np.float32)
    wv = rng.normal(size=(h, w)).astype(np.float32)
    sv = rng.uniform(size=(h, w)).astype(np.float32)
    bv = rng.normal(size=(h, w)).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    zd, wd, sd, bd, gd = (be.put(a) for a in (z, wv, sv, bv, g))
    G = L.nc_epilogue_fwd_partials(B, M, h, w)
    ws = be.zeros((L.nc_epilogue_workspace_size(B, M, h, w) // 4 + 1,))
    nb = ws.nbytes if hasattr(ws, "nbytes") else ws.numel() * 4
    aid = _abi.ACT_IDS["tanh"]
    out, parts = be.zeros((B, h, w)), be.zeros((G, B, h, w))
    mean, rstd = be.zeros((B, M)), be.zeros((B, M))
    _ok(be, L.nc_epilogue_fwd(s, B, M, h, w, aid, 0.01, 0, be.ptr(zd), None, be.ptr(wd),
                              be.ptr(sd), be.ptr(bd), be.ptr(out), be.ptr(mean), be.ptr(rstd),
                              be.ptr(ws), nb), "epi")
    _ok(be, L.nc_epilogue_fwd_parts(s, B, M, h, w, aid, 0.01, 0, be.ptr(zd), None, be.ptr(wd),
                                    be.ptr(sd), be.ptr(bd), be.ptr(parts), be.ptr(mean),
                                    be.ptr(rstd), be.ptr(ws), nb), "epi_parts")
    ph, pw = (kh - 1) // 2, (kw - 1) // 2
    ghat = be.zeros((M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_filter_spectrum_fwd(s, M, kh, kw, FH, FW, be.ptr(gd), be.ptr(ghat)), "spec")
    z1, x1 = be.zeros((B, M, h, w)), be.zeros((B, FH, FW // 2 + 1, 2))
    z2, x2 = be.zeros((B, M, h, w)), be.zeros((B, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_fftconv_fwd(s, B, M, h, w, h, w, ph, pw, FH, FW, be.ptr(out), be.ptr(ghat),
                             be.ptr(z1), be.ptr(x1)), "fwd")
    _ok(be, L.nc_fftconv_fwd_parts(s, B, M, h, w, h, w, ph, pw, FH, FW, be.ptr(parts), G, None,
                                   be.ptr(ghat), be.ptr(z2), be.ptr(x2)), "fwd_parts")
    o, p = be.get(out), be.get(parts)
    acc = p[0].copy()
    for q in range(1, G):
        acc = acc + p[q]
    o_r = O.epilogue_fwd(z, np.zeros((M, h, w), np.float32), wv, sv, bv, "tanh", False)[0]
    return {"G": G, "out": rel_l2(o, o_r),
            "parts_sum_mismatch": int((acc != o).sum()),
            "z_mismatch": int((be.get(z1) != be.get(z2)).sum()),
            "xhat_mismatch": int((be.get(x1) != be.get(x2)).sum())}


def case_fftconv_epilogue(be, B=3, M=6, h=20, w=27, kh=7, kw=5, FH=32, FW=64, act="tanh",
                          seed=8, two_pass=False):
    """nc_fftconv_spectra + nc_fftconv_epilogue_fwd (the fused correlation and hidden epilogue)
    against nc_fftconv_fwd_parts + nc_epilogue_fwd_parts and the oracle.  The cell state comes
    in two partial planes; M = 6 leaves two idle wavefronts in the last direction group; the
    call without z must give the same parts/mean/rstd bit for bit as the one with z.  With
    two_pass the workspace also holds nc_fftconv_correlate_workspace_size bytes, so a large
    grid's correlation runs as the two transform passes (the separate path keeps the
    segmented one)."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    ph, pw = (kh - 1) // 2, (kw - 1) // 2
    x = (rng.normal(size=(B, h, w)) * 0.7).astype(np.float32)
    x0 = (rng.normal(size=(B, h, w)) * 0.2).astype(np.float32)
    xp = np.stack([x0, x - x0])  # two partial planes; their fp32 sum is the state the kernels see
    xs = (xp[0] + xp[1]).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    wv = rng.normal(size=(h, w)).astype(np.float32)
    sv = rng.uniform(size=(h, w)).astype(np.float32)
    bv = rng.normal(size=(h, w)).astype(np.float32)
    xpd, gd, wd, sd, bd = (be.put(a) for a in (xp, g, wv, sv, bv))
    aid = _abi.ACT_IDS[act]
    ghat = be.zeros((M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_filter_spectrum_fwd(s, M, kh, kw, FH, FW, be.ptr(gd), be.ptr(ghat)), "spec")
    xh1, xh2 = be.zeros((B, FH, FW // 2 + 1, 2)), be.zeros((B, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_fftconv_spectra(s, B, h, w, FH, FW, be.ptr(xpd), 2, None, be.ptr(xh1)),
        "spectra")
    # the separate path: correlation (+ spectra) then the epilogue's partial outputs
    z_ref = be.zeros((B, M, h, w))
    _ok(be, L.nc_fftconv_fwd_parts(s, B, M, h, w, h, w, ph, pw, FH, FW, be.ptr(xpd), 2, None,
                                   be.ptr(ghat), be.ptr(z_ref), be.ptr(xh2)), "fwd_parts")
    Gs = L.nc_epilogue_fwd_partials(B, M, h, w)
    nws = L.nc_epilogue_workspace_size(B, M, h, w)
    if two_pass:
        assert L.nc_fftconv_correlate_workspace_size(B, M, h, w, FH, FW) > 0
        nws = max(nws, L.nc_fftconv_correlate_workspace_size(B, M, h, w, FH, FW))
    ws = be.zeros((nws // 4 + 1,))
    nb = ws.nbytes if hasattr(ws, "nbytes") else ws.numel() * 4
    p_ref, m_ref, r_ref = be.zeros((Gs, B, h, w)), be.zeros((B, M)), be.zeros((B, M))
    _ok(be, L.nc_epilogue_fwd_parts(s, B, M, h, w, aid, 0.01, 0, be.ptr(z_ref), None, be.ptr(wd),
                                    be.ptr(sd), be.ptr(bd), be.ptr(p_ref), be.ptr(m_ref),
                                    be.ptr(r_ref), be.ptr(ws), nb), "epi_parts")
    # the fused path, with and (on the fused grids) without z
    G = L.nc_fftconv_epilogue_partials(B, M, h, w, FH, FW)
    fused = FW == 64 and FH in (32, 64)
    z1 = be.zeros((B, M, h, w))
    outs = []
    for zz in ((z1, None) if fused else (z1,)):
        p, mu, rs = be.zeros((G, B, h, w)), be.zeros((B, M)), be.zeros((B, M))
        _ok(be, L.nc_fftconv_epilogue_fwd(s, B, M, h, w, ph, pw, FH, FW, be.ptr(xh1),
                                          be.ptr(ghat), aid, 0.01, be.ptr(wd), be.ptr(sd),
                                          be.ptr(bd), be.ptr(zz), be.ptr(p), be.ptr(mu),
                                          be.ptr(rs), be.ptr(ws), nb), "fused")
        outs.append(tuple(be.get(a) for a in (p, mu, rs)))
    p1, mu1, rs1 = outs[0]
    out1 = p1.astype(np.float64).sum(0)
    out_ref = be.get(p_ref).astype(np.float64).sum(0)
    zo = O.conv2d_direct(xs, g[:, 0], (ph, pw))
    o_or, m_or, r_or = O.epilogue_fwd(zo, np.zeros((M, h, w), np.float32), wv, sv, bv, act,
                                      False)
    res = {"G": G if fused else -1,
           "xhat_mismatch": int((be.get(xh1) != be.get(xh2)).sum()),
           "z": rel_l2(be.get(z1), zo),
           "z_vs_separate": rel_l2(be.get(z1), be.get(z_ref)),
           "out": rel_l2(out1, o_or),
           "out_vs_separate": rel_l2(out1, out_ref),
           "mean": rel_l2(mu1, m_or), "rstd": rel_l2(rs1, r_or)}
    if fused:
        res["no_z_mismatch"] = sum(int((a != b).sum()) for a, b in zip(outs[0], outs[1]))
    return res


def case_fused_forms(be, B_small, B_large, M=16, h=40, w=50, kh=23, kw=13, FH=64, FW=64,
                     act="tanh", seed=21):
    """The fused correlation + epilogue's two forms compute the same thing.  The launch takes
    the windowed form (the inverse's column pass keeps only the window's rows, zhat and act
    staged one plane at a time) when the grid holds more than two workgroups per CU, the
    full-row form otherwise; the same B_small samples run once alone (B_small * G at most
    twice the CU count) and once as the first samples of a B_large batch (above it).  Each
    sample's results depend on that sample only, so any difference is the forms': the
    full-row form's lanes hold runs of four pixels and the windowed form's single pixels, so
    their plane statistics are summed in different orders (and hipcc contracts the two
    compilations differently).  Returns the largest rel-L2 difference over z, the partial
    outputs, mean and rstd ("forms"), the elements that differ at all, and the windowed z
    against the oracle."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    ph, pw = (kh - 1) // 2, (kw - 1) // 2
    xs = (rng.normal(size=(B_small, h, w)) * 0.7).astype(np.float32)
    xl = np.concatenate([xs] + [(rng.normal(size=(B_large - B_small, h, w)) * 0.7)
                                .astype(np.float32)])
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32) / np.sqrt(kh * kw)
    wv = rng.normal(size=(h, w)).astype(np.float32)
    sv = rng.uniform(size=(h, w)).astype(np.float32)
    bv = rng.normal(size=(h, w)).astype(np.float32)
    gd, wd, sd, bd = (be.put(a) for a in (g, wv, sv, bv))
    aid = _abi.ACT_IDS[act]
    ghat = be.zeros((M, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_filter_spectrum_fwd(s, M, kh, kw, FH, FW, be.ptr(gd), be.ptr(ghat)), "spec")
    outs = []
    for x in (xs, xl):
        B = x.shape[0]
        xd = be.put(x)
        xh = be.zeros((B, FH, FW // 2 + 1, 2))
        _ok(be, L.nc_fftconv_spectra(s, B, h, w, FH, FW, be.ptr(xd), 1, None, be.ptr(xh)),
            "spectra")
        G = L.nc_fftconv_epilogue_partials(B, M, h, w, FH, FW)
        nws = L.nc_epilogue_workspace_size(B, M, h, w)
        ws = be.zeros((nws // 4 + 1,))
        nb = ws.nbytes if hasattr(ws, "nbytes") else ws.numel() * 4
        z, p = be.zeros((B, M, h, w)), be.zeros((G, B, h, w))
        mu, rs = be.zeros((B, M)), be.zeros((B, M))
        _ok(be, L.nc_fftconv_epilogue_fwd(s, B, M, h, w, ph, pw, FH, FW, be.ptr(xh),
                                          be.ptr(ghat), aid, 0.01, be.ptr(wd), be.ptr(sd),
                                          be.ptr(bd), be.ptr(z), be.ptr(p), be.ptr(mu),
                                          be.ptr(rs), be.ptr(ws), nb), "fused")
        outs.append((be.get(z)[:B_small], be.get(p)[:, :B_small], be.get(mu)[:B_small],
                     be.get(rs)[:B_small]))
    zo = O.conv2d_direct(xs, g[:, 0], (ph, pw))
    return {"forms": max(rel_l2(a, b) for a, b in zip(outs[0], outs[1])),
            "mismatch": sum(int((a != b).sum()) for a, b in zip(outs[0], outs[1])),
            "z": rel_l2(outs[1][0], zo)}


def case_fftconv_port(be, B=3, M=6, h=20, w=27, kh=7, kw=5, FH=32, FW=64, fact=None,
                      rows=(2, 3, 19, 3, 0), cols=(5, 5, 26, 5, 0), seed=11, two_pass=False):
    """nc_fftconv_port_fwd (the last step's correlation and output port in one operation)
    against nc_spectral_correlate + nc_port_fwd and the oracle: out, zo, mean, rstd, pre and z,
    with a duplicated port cell and the grid's corners; on the fused grids the call without z
    must give the same outputs bit for bit."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    ph, pw = (kh - 1) // 2, (kw - 1) // 2
    P = len(rows)
    idx = np.array([r * w + c for r, c in zip(rows, cols)], np.int32)
    x = rng.normal(size=(B, h, w)).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    pp = rng.normal(size=(3, P)).astype(np.float32)
    xd, gd, idd, ppd = be.put(x), be.put(g), be.put(idx, np.int32), be.put(pp)
    fid = _abi.ACT_IDS["identity" if fact is None else fact]
    ghat, xhat = be.zeros((M, FH, FW // 2 + 1, 2)), be.zeros((B, FH, FW // 2 + 1, 2))
    _ok(be, L.nc_filter_spectrum_fwd(s, M, kh, kw, FH, FW, be.ptr(gd), be.ptr(ghat)), "spec")
    _ok(be, L.nc_fftconv_spectra(s, B, h, w, FH, FW, be.ptr(xd), 1, None, be.ptr(xhat)), "xs")
    nws = L.nc_fftconv_port_workspace_size(B, M, h, w, FH, FW, P)
    if two_pass:  # room for the two-pass large-grid correlation as well
        assert L.nc_fftconv_correlate_workspace_size(B, M, h, w, FH, FW) > 0
        nws = max(nws, L.nc_fftconv_correlate_workspace_size(B, M, h, w, FH, FW))
    ws = be.zeros((nws // 4 + 1,))
    nb = ws.nbytes if hasattr(ws, "nbytes") else ws.numel() * 4
    res, got = {}, []
    fused = FW == 64 and FH in (32, 64)
    for mode in (("ref", "z", "noz") if fused else ("ref", "z")):
        out, zo = be.zeros((B, P)), be.zeros((B, M, P))
        mean, rstd, pre, z = be.zeros((B, M)), be.zeros((B, M)), be.zeros((B, P)), \
            be.zeros((B, M, h, w))
        if mode == "ref":
            _ok(be, L.nc_spectral_correlate(s, B, M, h, w, ph, pw, FH, FW, be.ptr(xhat),
                                            be.ptr(ghat), be.ptr(z)), "corr")
            _ok(be, L.nc_port_fwd(s, B, M, h, w, 0, fid, 0.01, P, be.ptr(idd), be.ptr(z), None,
                                  be.ptr(ppd), be.ptr(out), be.ptr(zo), be.ptr(mean),
                                  be.ptr(rstd), be.ptr(pre), be.ptr(ws), nb), "port")
        else:
            _ok(be, L.nc_fftconv_port_fwd(s, B, M, h, w, ph, pw, FH, FW, be.ptr(xhat),
                                          be.ptr(ghat), fid, 0.01, P, be.ptr(idd), be.ptr(ppd),
                                          be.ptr(z) if mode == "z" else None, be.ptr(out),
                                          be.ptr(zo), be.ptr(mean), be.ptr(rstd), be.ptr(pre),
                                          be.ptr(ws), nb), "fused")
        got.append({k: be.get(v) for k, v in (("out", out), ("zo", zo), ("mean", mean),
                                               ("rstd", rstd), ("pre", pre), ("z", z))})
    ref, fz = got[0], got[1]
    zr = O.conv2d_direct(x, g[:, 0], (ph, pw))
    o_r, aux = O.port_fwd(zr, np.zeros((M, h, w)), np.array(rows), np.array(cols), (P, 1),
                          pp[0][:, None], pp[1][:, None], pp[2][:, None], False, fact)
    res["out"] = rel_l2(fz["out"], o_r[:, :, 0])
    res["zo"] = rel_l2(fz["zo"], aux["zo"][..., 0])
    res["z"] = rel_l2(fz["z"], zr)
    for k in ("out", "zo", "mean", "rstd", "z") + (("pre",) if fact else ()):
        res[k + "_vs_separate"] = rel_l2(fz[k], ref[k])
    if fused:
        res["no_z_mismatch"] = float(sum(int((got[1][k] != got[2][k]).sum())
                                         for k in ("out", "zo", "mean", "rstd", "pre")))
    return res


def case_fftconv_circular(be, B=2, M=3, H=16, W=16, kh=5, kw=3, seed=9):
    """CIRCULAR padding mode (propagator.py:284-300): the correlation on the (H, W) grid itself,
    the output window read modulo the grid, forward (nc_fftconv_fwd and, on the 64-wide grids,
    the fused correlation + epilogue) and reverse (dx, dG) against the wrap-padded brute-force
    correlation and its adjoints."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    pad = ((kh - 1) // 2, (kw - 1) // 2)
    x = rng.normal(size=(B, H, W)).astype(np.float32)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    gz = rng.normal(size=(B, M, H, W)).astype(np.float32)
    xd, gd, gzd = be.put(x), be.put(g), be.put(gz)
    F2 = (M, H, W // 2 + 1, 2)
    ghat = be.zeros(F2)
    _ok(be, L.nc_filter_spectrum_fwd(s, M, kh, kw, H, W, be.ptr(gd), be.ptr(ghat)), "spec")
    z, xhat = be.zeros((B, M, H, W)), be.zeros((B, H, W // 2 + 1, 2))
    _ok(be, L.nc_fftconv_fwd(s, B, M, H, W, H, W, pad[0], pad[1], H, W, be.ptr(xd),
                             be.ptr(ghat), be.ptr(z), be.ptr(xhat)), "fwd")
    ws = be.zeros((L.nc_fftconv_bwd_workspace_size(B, M, H, W) // 4 + 1,))
    nb = ws.nbytes if hasattr(ws, "nbytes") else ws.numel() * 4
    dx, dgh = be.zeros((B, H, W)), be.zeros(F2)
    _ok(be, L.nc_fftconv_bwd(s, B, M, H, W, H, W, pad[0], pad[1], H, W, be.ptr(gzd),
                             be.ptr(xhat), be.ptr(ghat), 1, be.ptr(dx), be.ptr(dgh), 0, 0,
                             be.ptr(ws), nb), "bwd")
    gf = be.zeros((M, 1, kh, kw))
    _ok(be, L.nc_filter_spectrum_bwd(s, M, kh, kw, H, W, pad[0], pad[1], be.ptr(dgh),
                                     be.ptr(gf), 0, 0), "specbwd")
    zr = O.conv2d_circular_direct(x, g[:, 0], pad)
    dxr, dGh = O.conv2d_fft_unshifted_bwd(gz, x, g[:, 0], pad, (H, W))
    dgr = O.filter_grad_from_unshifted(dGh, (kh, kw), pad, (H, W))
    res = {"z": rel_l2(be.get(z), zr), "dx": rel_l2(be.get(dx), dxr),
           "dG": rel_l2(be.get(gf)[:, 0], dgr)}
    if W == 64 and H in (32, 64):
        wv = rng.normal(size=(H, W)).astype(np.float32)
        sv = rng.uniform(size=(H, W)).astype(np.float32)
        bv = rng.normal(size=(H, W)).astype(np.float32)
        wd, sd, bd = be.put(wv), be.put(sv), be.put(bv)
        G = L.nc_fftconv_epilogue_partials(B, M, H, W, H, W)
        p, mu, rs = be.zeros((G, B, H, W)), be.zeros((B, M)), be.zeros((B, M))
        z2 = be.zeros((B, M, H, W))
        _ok(be, L.nc_fftconv_epilogue_fwd(s, B, M, H, W, pad[0], pad[1], H, W, be.ptr(xhat),
                                          be.ptr(ghat), _abi.ACT_IDS["tanh"], 0.01, be.ptr(wd),
                                          be.ptr(sd), be.ptr(bd), be.ptr(z2), be.ptr(p),
                                          be.ptr(mu), be.ptr(rs), None, 0), "fused")
        o_r = O.epilogue_fwd(zr, np.zeros((M, H, W)), wv, sv, bv, "tanh", False)[0]
        res["z_fused"] = rel_l2(be.get(z2), zr)
        res["out_fused"] = rel_l2(be.get(p).astype(np.float64).sum(0), o_r)
    return res


def case_port(be, B=3, M=5, h=10, w=12, rows=(2, 3, 4, 2), cols=(5, 5, 5, 5), fact=None,
              seed=3, has_border=1):
    """Output-port forward/backward (rect-like and coordinate ports, duplicates included).
    Without the border term gdb must come back as exact zeros."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    P = len(rows)
    idx = np.array([r * w + c for r, c in zip(rows, cols)], np.int32)
    z = rng.normal(size=(B, M, h, w)).astype(np.float32)
    d = rng.normal(size=(M, h, w)).astype(np.float32)
    pp = rng.normal(size=(3, P)).astype(np.float32)
    go = rng.normal(size=(B, P)).astype(np.float32)
    idd, zd, dd, ppd, god = be.put(idx, np.int32), be.put(z), be.put(d), be.put(pp), be.put(go)
    out, zo = be.zeros((B, P)), be.zeros((B, M, P))
    mean, rstd, pre = be.zeros((B, M)), be.zeros((B, M)), be.zeros((B, P))
    ws = be.zeros((L.nc_epilogue_workspace_size(B, M, h, w) // 4 + 1,))
    nb = ws.nbytes if hasattr(ws, "nbytes") else ws.numel() * 4
    fid = _abi.ACT_IDS["identity" if fact is None else fact]
    hb = int(has_border)
    dptr = be.ptr(dd) if hb else None
    _ok(be, L.nc_port_fwd(s, B, M, h, w, hb, fid, 0.01, P, be.ptr(idd), be.ptr(zd), dptr,
                          be.ptr(ppd), be.ptr(out), be.ptr(zo), be.ptr(mean), be.ptr(rstd),
                          be.ptr(pre), be.ptr(ws), nb), "portf")
    gz, gpp = be.zeros((B, M, h, w)), be.zeros((3, P))
    gdb = be.put(np.full((M, h, w), 7.0, np.float32))
    _ok(be, L.nc_port_bwd(s, B, M, h, w, hb, fid, 0.01, P, be.ptr(idd), be.ptr(zd), dptr,
                          be.ptr(ppd), be.ptr(zo), be.ptr(mean), be.ptr(rstd), be.ptr(pre),
                          be.ptr(god), be.ptr(gz), be.ptr(gdb), be.ptr(gpp), 0, be.ptr(ws), nb),
        "portb")
    R, Cc = np.array(rows), np.array(cols)
    o_r, aux = O.port_fwd(z, d, R, Cc, (P, 1), pp[0][:, None], pp[1][:, None], pp[2][:, None],
                          bool(hb), fact)
    r = O.port_bwd(z, d, R, Cc, (P, 1), pp[0][:, None], pp[1][:, None], pp[2][:, None], aux,
                   go[:, :, None], bool(hb), fact)
    g = be.get(gpp)
    # the row-stack variant (padded plane stride), summed by nc_rows_sum: the same reduction
    # over the same rows, so bit for bit the same gradients
    stride = B * P + 7
    prow, gz2, gpp2 = be.zeros((3 * stride,)), be.zeros((B, M, h, w)), be.zeros((3, P))
    _ok(be, L.nc_port_bwd_parts(s, B, M, h, w, hb, fid, 0.01, P, be.ptr(idd), be.ptr(zd),
                                dptr, be.ptr(ppd), be.ptr(zo), be.ptr(mean), be.ptr(rstd),
                                be.ptr(pre), be.ptr(god), be.ptr(gz2), be.ptr(prow), stride,
                                be.ptr(ws), nb), "portb_parts")
    a = lambda t, off=0: be.ptr(t).value + 4 * off
    jobs = _abi.rows_jobs(*[(a(prow, i * stride), a(gpp2, i * P), P, 0, B) for i in range(3)])
    _ok(be, L.nc_rows_sum(s, 3, jobs), "rows_sum")
    return {"out": rel_l2(be.get(out), o_r[:, :, 0]), "zo": rel_l2(be.get(zo), aux["zo"][..., 0]),
            "gz": rel_l2(be.get(gz), r[0]),
            ("gdb" if hb else "gdb_nonzero"): (rel_l2(be.get(gdb), r[1]) if hb else
                                               float((be.get(gdb) != 0.0).sum())),
            "gw_out": rel_l2(g[0], r[2][:, 0]), "gs_out": rel_l2(g[1], r[3][:, 0]),
            "gb_out": rel_l2(g[2], r[4][:, 0]),
            "parts_gz_mismatch": float((be.get(gz2) != be.get(gz)).sum()),
            "parts_gpp_mismatch": float((be.get(gpp2) != g).sum())}


def case_codd(be, mode="continuous", bbox=None, hard_pin=0, tau=0.1, seed=4):
    """Pre-step Codd fusion forward and reverse on the ALU geometry (16-cell output port)."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    geom = O.alu_geometry(out_width=2)
    H, W = geom.grid_shape
    kh, kw = geom.kernel_size
    M = geom.directions
    cell = (rng.normal(size=(3, H, W)) * np.array([0.1, 0.3, 1.0])[:, None, None]).astype(
        np.float32)
    rows, cols = geom.out_cells_roi
    P = len(rows)
    r0, r1, c0, c1 = bbox or (0, geom.roi_shape[0], 0, geom.roi_shape[1])
    chip = _abi.ChipDesc(H, W, kh, kw, M, geom.pad_h, geom.pad_w, *geom.roi_shape, r0, r1, c0, c1)
    h, w = r1 - r0, c1 - c0
    cd = be.put(cell)
    io = be.put(geom.io_state_mask, np.uint8)
    owm = be.put(geom.out_weight_mask, np.uint8)
    prc = be.put(np.stack([rows, cols]), np.int32)
    we, se, br = be.zeros((h, w)), be.zeros((h, w)), be.zeros((h, w))
    patch, pp = be.zeros((h + kh - 1, w + kw - 1)), be.zeros((3, P))
    sp_, b2d, wp = be.zeros((H, W)), be.zeros((H, W)), be.zeros((H, W))
    mid, it = _abi.CODD_IDS[mode], O.inv_tau_f32(tau)
    _ok(be, L.nc_codd_fuse_fwd(s, C.byref(chip), be.ptr(cd), be.ptr(io), be.ptr(owm), mid, it,
                               0.6, hard_pin, 1, 0.01, P, be.ptr(prc), be.ptr(we), be.ptr(se),
                               be.ptr(br), be.ptr(patch), be.ptr(pp), be.ptr(sp_), be.ptr(b2d),
                               be.ptr(wp)), "codd")
    # the fused prologue: the same Codd results bit for bit, and the injection's gather
    Bi, n_in = 2, 7
    src = rng.integers(-1, n_in, size=h * w).astype(np.int32)
    xin = rng.normal(size=(Bi, n_in)).astype(np.float32)
    srcd, xind, roi = be.put(src, np.int32), be.put(xin), be.zeros((Bi, h * w))
    f2 = [be.zeros(np.shape(a)) for a in (we, se, br, patch, pp, sp_)]
    _ok(be, L.nc_step_prologue(s, C.byref(chip), be.ptr(cd), be.ptr(io), be.ptr(owm), mid, it,
                               0.6, hard_pin, 1, 0.01, P, be.ptr(prc),
                               *[be.ptr(a) for a in f2], Bi, n_in, be.ptr(xind), h * w,
                               be.ptr(srcd), be.ptr(roi)), "prologue")
    pro_ref = np.where(src >= 0, xin[:, np.maximum(src, 0)], 0.0)
    pro_bad = sum(int((be.get(a) != be.get(b_)).sum())
                  for a, b_ in zip(f2, (we, se, br, patch, pp, sp_)))
    pro_bad += int((be.get(roi) != pro_ref).sum())
    sp = O.precompute_step_params(cell, geom, "tanh", bool(hard_pin), bbox, mode, tau, 0.6)
    fwd_got = np.concatenate([be.get(a).ravel() for a in (we, se, br, patch, pp)])
    fwd_ref = np.concatenate([np.ravel(a) for a in (
        sp["w_eff_roi"], sp["s_eff_roi"], sp["b_roi"], O.border_patch(sp["border_2d"], geom, bbox),
        sp["w_eff_out"], sp["s_eff_out"], sp["b_out"])])
    gi = [rng.normal(size=(h, w)).astype(np.float32) for _ in range(3)]
    gpatch = rng.normal(size=(h + kh - 1, w + kw - 1)).astype(np.float32)
    gpp = rng.normal(size=(3, P)).astype(np.float32)
    gid = [be.put(a) for a in gi]
    gpd, gppd = be.put(gpatch), be.put(gpp)
    gsp, gbf = (rng.normal(size=(H, W)).astype(np.float32) for _ in range(2))
    gspd, gbfd = be.put(gsp), be.put(gbf)  # held: a device tensor must outlive the launch
    gcell = be.zeros((3, H, W))
    _ok(be, L.nc_codd_fuse_bwd(s, C.byref(chip), be.ptr(cd), be.ptr(io), be.ptr(owm), mid, it,
                               0.6, hard_pin, 1, 0.01, P, be.ptr(prc), None, None,
                               *[be.ptr(a) for a in gid], be.ptr(gpd), be.ptr(gppd), be.ptr(gspd),
                               be.ptr(gbfd), be.ptr(gcell)), "coddb")
    # the same with the ports listed by ROI cell (the step executor's form): equal bit for bit
    prc_h = be.get(prc).astype(np.int64)
    cell_of = prc_h[0] * geom.roi_shape[1] + prc_h[1]
    order = np.argsort(cell_of, kind="stable")
    start = np.searchsorted(cell_of[order], np.arange(geom.roi_shape[0] * geom.roi_shape[1] + 1))
    std, lsd = be.put(start.astype(np.int32), np.int32), be.put(order.astype(np.int32), np.int32)
    gcell2 = be.zeros((3, H, W))
    _ok(be, L.nc_codd_fuse_bwd(s, C.byref(chip), be.ptr(cd), be.ptr(io), be.ptr(owm), mid, it,
                               0.6, hard_pin, 1, 0.01, P, be.ptr(prc), be.ptr(std), be.ptr(lsd),
                               *[be.ptr(a) for a in gid], be.ptr(gpd), be.ptr(gppd), be.ptr(gspd),
                               be.ptr(gbfd), be.ptr(gcell2)), "coddb_csr")
    pro_bad += int((be.get(gcell2) != be.get(gcell)).sum())
    gbd = np.zeros((H, W))
    gbd[r0:r0 + gpatch.shape[0], c0:c0 + gpatch.shape[1]] = gpatch
    gbd[geom.pad_h:H - geom.pad_h, geom.pad_w:W - geom.pad_w] = 0
    oh, ow = geom.out_size
    ref = O.precompute_step_params_vjp(
        cell, geom, dict(w_eff_roi=gi[0], s_eff_roi=gi[1], b_roi=gi[2], border_2d=gbd,
                         w_eff_out=gpp[0].reshape(oh, ow), s_eff_out=gpp[1].reshape(oh, ow),
                         b_out=gpp[2].reshape(oh, ow), s_prob=gsp, b_full=gbf),
        "tanh", bool(hard_pin), bbox, mode, tau, 0.6)
    return {"fwd": rel_l2(fwd_got, fwd_ref), "s_prob": rel_l2(be.get(sp_), sp["s_prob"]),
            "border_2d": rel_l2(be.get(b2d), sp["border_2d"]),
            "w_pinned": rel_l2(be.get(wp), sp["w_pinned"]), "g_cell": rel_l2(be.get(gcell), ref),
            "prologue_mismatch": float(pro_bad)}


def case_universe(be, pmode="VALID", bbox=None, fact="tanh", B=3, G=2, seed=10):
    """nc_universe_fwd / nc_universe_bwd: the final universe and the full-grid port read from
    it (propagator.py:684-734), with a port on the border and a cell read twice."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    out = ("coords", [(0, 0), (1, 5), (8, 7), (15, 13), (6, 9), (8, 7)])
    geom = O.Geometry((16, 14), (5, 3), 3, 2, [("rect", (5, 3), (4, 1))], out,
                      padding_mode=pmode)
    H, W = geom.grid_shape
    r0, r1, c0, c1 = bbox or (0, geom.roi_shape[0], 0, geom.roi_shape[1])
    h, w = r1 - r0, c1 - c0
    chip = _abi.ChipDesc(H, W, 5, 3, 3, geom.pad_h, geom.pad_w, *geom.roi_shape, r0, r1, c0, c1)
    parts = rng.normal(0, 0.7, size=(G, B, h, w)).astype(np.float32)
    bf = rng.normal(size=(H, W)).astype(np.float32)
    sp = rng.random((H, W)).astype(np.float32)
    gr, gc = geom.out_cells_grid
    cells = (gr * W + gc).astype(np.int32)
    P = cells.size
    head, nxt = np.full(H * W, -1, np.int32), np.full(P, -1, np.int32)
    for k in range(P - 1, -1, -1):
        nxt[k], head[cells[k]] = head[cells[k]], k
    valid = int(pmode == "VALID")
    fid, slope = _abi.ACT_IDS[fact or "identity"], 0.01
    # every operand held in a name: a device tensor must outlive the launch
    pd, bfd, spd = be.put(parts), be.put(bf), be.put(sp)
    cd, hd, nd = be.put(cells, np.int32), be.put(head, np.int32), be.put(nxt, np.int32)
    univ, outd = be.zeros((B, H, W)), be.zeros((B, P))
    _ok(be, L.nc_universe_fwd(s, C.byref(chip), B, G, valid, fid, slope, be.ptr(pd),
                              be.ptr(bfd), be.ptr(spd), P, be.ptr(cd), be.ptr(univ),
                              be.ptr(outd)), "universe_fwd")
    sp_d = dict(b_full=bf.astype(np.float64), s_prob=sp.astype(np.float64))
    ref_u, pre = O.universe_embed(parts.astype(np.float64).sum(0), sp_d, geom, fact, bbox)
    g_out = rng.normal(size=(B, P)).astype(np.float32)
    g_u = rng.normal(size=(B, H, W)).astype(np.float32)
    god, gud = be.put(g_out), be.put(g_u)
    g_roi, gsp, gbf = be.zeros((B, h, w)), be.zeros((H, W)), be.zeros((H, W))
    _ok(be, L.nc_universe_bwd(s, C.byref(chip), B, G, valid, fid, slope, be.ptr(pd),
                              be.ptr(bfd), be.ptr(spd), P, be.ptr(hd), be.ptr(nd), be.ptr(god),
                              be.ptr(gud), be.ptr(g_roi), be.ptr(gsp) if valid else None,
                              be.ptr(gbf) if valid else None), "universe_bwd")
    ref_g, extra = O.universe_vjp(pre, g_out, g_u, sp_d, geom, fact, bbox)
    res = {"universe": rel_l2(be.get(univ), ref_u),
           "out": rel_l2(be.get(outd), ref_u[:, gr, gc]),
           "g_roi": rel_l2(be.get(g_roi), ref_g)}
    if valid:
        res["g_s_prob"] = rel_l2(be.get(gsp), extra["s_prob"])
        res["g_b_full"] = rel_l2(be.get(gbf), extra["b_full"])
    return res


def case_adaptive(be, seed=5):
    """Adaptive-mask statistics: the 8 integers and the dilated mask are compared exactly
    (returned as mismatch counts)."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    geom = O.alu_geometry(out_width=2)
    H, W = geom.grid_shape
    kh, kw = geom.kernel_size
    M = geom.directions
    hv, wv = geom.roi_shape
    cell = (rng.normal(size=(3, H, W)) * np.array([0.1, 0.3, 1.0])[:, None, None]).astype(
        np.float32)
    cell[1, 20, 30], cell[2, 20, 30] = 0.8, 2.0
    env = np.exp(-((np.arange(kh)[:, None] - 11) ** 2 / 8.0 + (np.arange(kw)[None] - 6) ** 2 / 4.0))
    filt = (rng.normal(size=(M, 1, kh, kw)) * env[None, None]).astype(np.float32)
    chip = _abi.ChipDesc(H, W, kh, kw, M, geom.pad_h, geom.pad_w, hv, wv, 0, hv, 0, wv)
    io_roi = geom.io_state_mask[geom.pad_h:H - geom.pad_h, geom.pad_w:W - geom.pad_w]
    st, dil = be.zeros((8,), np.int32), be.zeros((hv, wv), np.uint8)
    # operands stay referenced until the (asynchronous) launch has completed
    cd, fd, iod = be.put(cell), be.put(filt), be.put(io_roi, np.uint8)
    _ok(be, L.nc_adaptive_stats(s, C.byref(chip), be.ptr(cd), be.ptr(fd), be.ptr(iod), None, 4, 4,
                                2.5, 0.05, 0.05, 1e-3, be.ptr(st), be.ptr(dil)), "adaptive")
    st_r, dil_r = O.adaptive_mask_stats(cell, filt, io_roi, geom, (4, 4))
    return {"stats_mismatch": float((be.get(st) != st_r).sum()),
            "mask_mismatch": float((be.get(dil).astype(bool) != dil_r).sum())}


def case_spectral_ops(be, n=3, FH=32, FW=16, roi=(12, 10), pad=(5, 3), shift=(7, 5), seed=11):
    """nc_spectrum_map (phase ramp, Hermitian edge parts, column scales, conjugation),
    nc_irfft2_pruned on non-Hermitian spectra (NumPy's inverse keeps only the edge columns'
    Hermitian parts) and nc_standardize_fwd/bwd against float64 NumPy."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    Fh = FW // 2 + 1
    X = rng.normal(size=(n, FH, Fh)) + 1j * rng.normal(size=(n, FH, Fh))
    Xf = np.stack([X.real, X.imag], -1).astype(np.float32)
    xd = be.put(Xf)
    out = be.zeros((n, FH, Fh, 2))
    # conj, herm edges, scales 0.5 / 2, phase of a circular shift
    _ok(be, L.nc_spectrum_map(s, n, FH, FW, shift[0], shift[1], 1, 0.5, 2.0, 1, be.ptr(xd),
                              be.ptr(out)), "spectrum_map")
    Y = np.conj(X)
    H = Y.copy()
    for c in (0, FW // 2):
        H[:, :, c] = 0.5 * (Y[:, :, c] + np.conj(Y[:, (-np.arange(FH)) % FH, c]))
    scale = np.full(Fh, 2.0)
    scale[[0, -1]] = 0.5
    kh, kw = np.arange(FH)[:, None], np.arange(Fh)[None, :]
    phase = np.exp(-2j * np.pi * (kh * shift[0] / FH + kw * shift[1] / FW))
    ref_map = H * scale * phase
    res = {"spectrum_map": rel_l2(_cplx(be.get(out)), ref_map)}
    # the phase ramp equals the spectrum of the circularly shifted plane
    pl = rng.normal(size=(FH, FW))
    P = np.fft.rfft2(pl)
    pd, po = be.put(np.stack([P.real, P.imag], -1)), be.zeros((1, FH, Fh, 2))
    _ok(be, L.nc_spectrum_map(s, 1, FH, FW, shift[0], shift[1], 0, 1.0, 1.0, 0, be.ptr(pd),
                              be.ptr(po)), "spectrum_map_shift")
    res["phase_is_shift"] = rel_l2(_cplx(be.get(po))[0], np.fft.rfft2(np.roll(pl, shift, (0, 1))))
    # irfft2_pruned
    rh, rw = roi
    z = be.zeros((n, rh, rw))
    ws = be.zeros((L.nc_irfft2_pruned_workspace_size(n, FH, FW) // 4 + 1,))
    nb = ws.nbytes if hasattr(ws, "nbytes") else ws.numel() * 4
    _ok(be, L.nc_irfft2_pruned(s, n, rh, rw, pad[0], pad[1], FH, FW, be.ptr(xd), be.ptr(z),
                               be.ptr(ws), nb), "irfft2_pruned")
    full = np.fft.irfft2(X, s=(FH, FW))
    res["irfft2_pruned"] = rel_l2(be.get(z), full[:, pad[0]:pad[0] + rh, pad[1]:pad[1] + rw])
    # standardize
    planes, npx = 5, 7 * 9
    x = (rng.normal(size=(planes, npx)) * 2 + 1).astype(np.float32)
    g = rng.normal(size=(planes, npx)).astype(np.float32)
    xd2, gd = be.put(x), be.put(g)
    o, mu, rs, gx = (be.zeros((planes, npx)), be.zeros((planes,)), be.zeros((planes,)),
                     be.zeros((planes, npx)))
    _ok(be, L.nc_standardize_fwd(s, planes, npx, be.ptr(xd2), be.ptr(o), be.ptr(mu),
                                 be.ptr(rs)), "std_fwd")
    _ok(be, L.nc_standardize_bwd(s, planes, npx, be.ptr(xd2), be.ptr(mu), be.ptr(rs),
                                 be.ptr(gd), be.ptr(gx)), "std_bwd")
    x64 = x.astype(np.float64)
    m = x64.mean(-1, keepdims=True)
    r = 1.0 / np.sqrt(((x64 - m) ** 2).mean(-1, keepdims=True) + 1e-5)
    zh = (x64 - m) * r
    c1, c2 = g.mean(-1, keepdims=True), (g * zh).mean(-1, keepdims=True)
    res["std_fwd"] = rel_l2(be.get(o), zh)
    res["std_rstd"] = rel_l2(be.get(rs), r[:, 0])
    res["std_bwd"] = rel_l2(be.get(gx), r * (g - c1 - zh * c2))
    return res


def case_direct_conv(be, B=3, M=5, H=12, W=14, kh=3, kw=3, mode="SAME", n_parts=2, seed=12):
    """Direct small-filter correlation forward, input and filter gradients against the
    oracle's brute-force correlations: SAME (zero padding), VALID and CIRCULAR (wrap), with
    the input given as partial planes."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    parts = rng.normal(size=(n_parts, B, H, W)).astype(np.float32)
    x = parts.astype(np.float64).sum(0)
    g = rng.normal(size=(M, 1, kh, kw)).astype(np.float32)
    if mode == "VALID":
        ho, wo, oh, ow = H - kh + 1, W - kw + 1, 0, 0
    else:
        ho, wo, oh, ow = H, W, -((kh - 1) // 2), -((kw - 1) // 2)
    circ = int(mode == "CIRCULAR")
    gz = rng.normal(size=(B, M, ho, wo)).astype(np.float32)
    xd, gd, gzd = be.put(parts), be.put(g), be.put(gz)
    z, dx = be.zeros((B, M, ho, wo)), be.zeros((B, H, W))
    R = L.nc_direct_conv_dg_partials(B, M, ho, wo, kh, kw)
    part = be.zeros((R, M * kh * kw))
    _ok(be, L.nc_direct_conv_fwd(s, B, M, H, W, ho, wo, oh, ow, kh, kw, circ, be.ptr(xd),
                                 n_parts, be.ptr(gd), be.ptr(z)), "dconv_fwd")
    _ok(be, L.nc_direct_conv_bwd(s, B, M, H, W, ho, wo, oh, ow, kh, kw, circ, be.ptr(gzd),
                                 be.ptr(xd), n_parts, be.ptr(gd), 1, be.ptr(dx), be.ptr(part)),
        "dconv_bwd")
    dg = be.zeros((M * kh * kw,))
    a = lambda t: be.ptr(t).value
    _ok(be, L.nc_rows_sum(s, 1, _abi.rows_jobs((a(part), a(dg), M * kh * kw, 0, R))), "rows_sum")
    with O.precision(np.float64):
        if mode == "CIRCULAR":
            r_z = O.conv2d_circular_direct(x, g[:, 0], (-oh, -ow))
            # the circular correlation's adjoints: the same wrap on the padded input
            xp = np.pad(x, ((0, 0), (-oh, -oh), (-ow, -ow)), mode="wrap")
            r_dxp, r_dg = O.conv2d_bwd_direct(gz, xp, g[:, 0], (0, 0))
            r_dx = np.zeros_like(x)
            Hp, Wp = xp.shape[1:]
            for i in range(Hp):
                for j in range(Wp):
                    r_dx[:, (i + oh) % H, (j + ow) % W] += r_dxp[:, i, j]
        else:
            r_z = O.conv2d_direct(x, g[:, 0], (-oh, -ow))
            r_dx, r_dg = O.conv2d_bwd_direct(gz, x, g[:, 0], (-oh, -ow))
    return {"z": rel_l2(be.get(z), r_z), "dx": rel_l2(be.get(dx), r_dx),
            "dg": rel_l2(be.get(dg).reshape(M, kh, kw), r_dg)}


def case_helpers(be, seed=6):
    """Input injection (exact), MSE loss and three AdamW steps."""
    rng = np.random.default_rng(seed)
    L, s = be.lib, be.stream()
    B, n_in, n_roi = 4, 24, 200
    inp = rng.normal(size=(B, n_in)).astype(np.float32)
    src = np.full(n_roi, -1, np.int32)
    src[[5, 77, 199]] = [0, 3, 23]
    roi = be.zeros((B, n_roi))
    inpd, srcd = be.put(inp), be.put(src, np.int32)
    _ok(be, L.nc_inject_roi(s, B, n_in, be.ptr(inpd), n_roi, be.ptr(srcd), be.ptr(roi)), "inject")
    ref = np.zeros((B, n_roi), np.float32)
    ref[:, [5, 77, 199]] = inp[:, [0, 3, 23]]
    pr = rng.normal(size=100).astype(np.float32)
    tg = rng.normal(size=100).astype(np.float32)
    loss, gp = be.zeros((1,)), be.zeros((100,))
    prd, tgd = be.put(pr), be.put(tg)
    _ok(be, L.nc_mse_loss(s, 100, be.ptr(prd), be.ptr(tgd), be.ptr(loss), be.ptr(gp)), "mse")
    l_r, g_r = O.mse_loss(pr, tg)
    # a two-entry schedule table: steps 0 and >=1 use 0.01 and 0.02
    lr_tab = np.array([0.01, 0.02], np.float32)
    lr = be.put(lr_tab)
    res = {"inject_mismatch": float((be.get(roi) != ref).sum()),
           "mse": abs(float(be.get(loss)[0]) - l_r) / l_r, "g_mse": rel_l2(be.get(gp), g_r)}
    # one workgroup (small vectors) and the grid-wide update plus counter launch (large)
    for n, tag in ((50, ""), (70000, "_large")):
        p0 = rng.normal(size=n).astype(np.float32)
        g = rng.normal(size=n).astype(np.float32)
        p, gd = be.put(p0), be.put(g)
        m, v, cnt = be.zeros((n,)), be.zeros((n,)), be.zeros((1,), np.int32)
        pr_, mr, vr, cr = p0.astype(np.float64), 0.0, 0.0, 0
        for k in range(3):
            _ok(be, L.nc_adamw_step(s, n, be.ptr(p), be.ptr(gd), be.ptr(m), be.ptr(v),
                                    be.ptr(cnt), be.ptr(lr), 2, 0.9, 0.999, 1e-8, 1e-4), "adamw")
            pr_, mr, vr, cr = O.adamw_step(pr_, g.astype(np.float64), mr, vr, cr,
                                           float(lr_tab[min(k, 1)]))
        res["adamw" + tag] = rel_l2(be.get(p), pr_)
        res["count_mismatch" + tag] = float(be.get(cnt)[0] != 3)
    res["count_mismatch"] += res.pop("count_mismatch_large")
    return res


EPILOGUE_SHAPES = [
    # (B, M, h, w, act, has_border): single pass, tiled Chan (> 8192 px, partial last tile)
    (3, 5, 10, 12, "tanh", 1),
    (2, 16, 40, 50, "tanh", 0),
    (2, 3, 24, 32, "sigmoid", 1),
    (2, 4, 20, 40, "leaky_relu", 1),
    (2, 3, 33, 47, "relu", 1),
    (2, 3, 96, 100, "gelu", 1),
    (1, 2, 90, 92, "identity", 0),
    (2, 3, 91, 91, "tanh", 1),  # tiled with N % 4 != 0: the per-pixel (non-vector) tiles
]

PORT_SHAPES = [
    # (B, M, h, w, rows, cols, final activation, has_border)
    (3, 5, 10, 12, (2, 3, 4, 2), (5, 5, 5, 5), None, 1),
    (2, 16, 40, 50, tuple(range(16, 24)) * 2, (35,) * 8 + (36,) * 8, None, 1),
    (2, 3, 96, 100, (10, 50, 95), (3, 99, 0), "tanh", 1),
    (3, 4, 12, 10, (1, 7, 7), (2, 3, 3), "sigmoid", 0),
]

CODD_CASES = [(m, b, hp) for m in O.CODD_MODES for b in (None, (6, 30, 10, 42)) for hp in (0, 1)]

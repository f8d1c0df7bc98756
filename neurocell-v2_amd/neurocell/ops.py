"""Operator layer: the reference's custom-VJP operators as torch autograd Functions over the
gfx950 C ABI, with the reference's names, positional signatures, residuals and cotangents.

=========================================  ===============================================
reference operator (file:line)             here
=========================================  ===============================================
pallas_fused_roi_step_epilogue             ``pallas_fused_roi_step_epilogue`` (epilogue
  kernels_pallas.py:663-1069                 kernels, nc_epilogue_fwd/bwd)
fused_roi_step_epilogue epilogue.py:28-56  same kernels (norm=True)
pallas_fused_output_port_epilogue          ``pallas_fused_output_port_epilogue``
  kernels_pallas.py:1510-1551                (nc_port_fwd/bwd, grads to the port params)
fused_output_port_epilogue :82-128         same kernels (norm=True)
pallas_standardize_output_port             ``pallas_standardize_output_port`` (port kernels,
  kernels_pallas.py:1256-1507                standardisation-only mode)
precompute_filter_rfft2 greens:240-259     ``precompute_filter_rfft2`` (nc_filter_spectrum_fwd)
hoist_filter_rfft2_nopad pallas:1582-1604  ``hoist_filter_rfft2_nopad`` (bwd: roll by pad)
hoist_filter_rfft2_zero_nopad :1607-1631   ``hoist_filter_rfft2_zero_nopad``
rfft2_unshifted_filter_grad_to_oihw        ``rfft2_unshifted_filter_grad_to_oihw``
  kernels_pallas.py:1558-1579                (nc_filter_spectrum_bwd)
conv2d_pruned_rfft_roi_step :1759-1826     ``conv2d_pruned_rfft_roi_step`` (nc_fftconv_*)
conv2d_hybrid_nopad_roi_step :1634-1697    ``conv2d_hybrid_nopad_roi_step``
conv2d_small_kernel_roi_step :1700-1756    ``conv2d_small_kernel_roi_step``
conv2d_batched_nchw greens:177-217         ``conv2d_batched_nchw`` (VALID / SAME, via the
                                             spectral correlation)
rfft2_pruned / irfft2_pruned greens:25-66  ``rfft2_pruned`` (nc_plane_spectrum),
                                             ``irfft2_pruned`` (nc_irfft2_pruned); each the
                                             other's adjoint up to column weights
conv2d_grouped_filter_grad greens:84-123   ``conv2d_grouped_filter_grad`` (the Plancherel
                                             dG: nc_fftconv_bwd + nc_filter_spectrum_bwd)
rfft2_filter_grad_to_oihw greens:262-275   ``rfft2_filter_grad_to_oihw``
hoist_filter_rfft2 greens:278-313          ``hoist_filter_rfft2`` (bwd without a roll)
conv2d_roi_rfft_step greens:316-400        ``conv2d_roi_rfft_step`` (shifted cotangent:
                                             nc_spectrum_map of the unshifted one)
conv2d_valid_rfft_precomputed :403-425     ``conv2d_valid_rfft_precomputed``
hoist_filter_rfft2_zero_fwd :428-465       ``hoist_filter_rfft2_zero_fwd``
conv2d_hybrid_roi_step greens:468-551      ``conv2d_hybrid_roi_step``
standardize_spatial_nchw epilogue.py:20-25 ``standardize_spatial_nchw`` (nc_standardize_*)
fused_roi_epilogue epilogue.py:59-79       ``fused_roi_epilogue``
=========================================  ===============================================

Complex spectra are complex64 tensors (interleaved re/im, the C ABI's layout).  Autograd
cotangents of complex tensors follow PyTorch's convention (the conjugate of JAX's); the
kernels take a flag for it, so a chain conv -> hoist backward is bit-for-bit the reference's
unshifted Plancherel pairing.
"""
from __future__ import annotations

import torch

from . import _abi
from ._lib import NeurocellError, call, lib, ptr, stream_ptr
from .engine import act_id, spectral_grid_supported
from .topology import ChipTopology2D, CoordinatePortSpec



def _npow2(x):
    return 1 << (int(x) - 1).bit_length()


def _f32(t):
    if not t.is_cuda or t.dtype != torch.float32:
        raise NeurocellError("expected a float32 device tensor")
    return t.contiguous()


def _ws(nbytes, device):
    return torch.empty(max(1, (int(nbytes) + 3) // 4), device=device, dtype=torch.float32)


def is_supported_pallas_activation(activate) -> bool:
    """kernels_pallas.py:102-108."""
    try:
        act_id(activate)
        return True
    except ValueError:
        return False


# ------------------------------------------------------------------ hidden-step epilogue

class _Epilogue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, z, delta, w, s, b, act, slope, has_border):
        z, w, s, b = _f32(z), _f32(w), _f32(s), _f32(b)
        B, M, h, wd = z.shape
        d = _f32(delta).reshape(M, h, wd) if has_border else delta.contiguous()
        out = torch.empty(B, h, wd, device=z.device, dtype=torch.float32)
        mean = torch.empty(B, M, device=z.device, dtype=torch.float32)
        rstd = torch.empty_like(mean)
        L = lib()
        ws = _ws(L.nc_epilogue_workspace_size(B, M, h, wd), z.device)
        call("nc_epilogue_fwd", stream_ptr(), B, M, h, wd, act, slope, int(has_border), ptr(z),
             ptr(d) if has_border else None, ptr(w), ptr(s), ptr(b), ptr(out), ptr(mean),
             ptr(rstd), ptr(ws), ws.numel() * 4)
        ctx.save_for_backward(z, d, w, s, b, mean, rstd)
        ctx.args = (act, slope, has_border, tuple(delta.shape))
        return out

    @staticmethod
    def backward(ctx, gy):
        z, d, w, s, b, mean, rstd = ctx.saved_tensors
        act, slope, hb, dshape = ctx.args
        B, M, h, wd = z.shape
        gz = torch.empty_like(z)
        gdb = torch.zeros(M, h, wd, device=z.device, dtype=torch.float32)
        gw, gs, gb = (torch.empty(h, wd, device=z.device, dtype=torch.float32) for _ in range(3))
        L = lib()
        ws = _ws(L.nc_epilogue_workspace_size(B, M, h, wd), z.device)
        call("nc_epilogue_bwd", stream_ptr(), B, M, h, wd, act, slope, int(hb), ptr(z),
             ptr(d) if hb else None, ptr(w), ptr(s), ptr(b), ptr(mean), ptr(rstd),
             ptr(_f32(gy)), ptr(gz), ptr(gdb) if hb else None, ptr(gw), ptr(gs), ptr(gb), 0, 0,
             ptr(ws), ws.numel() * 4)
        return gz, gdb.reshape(dshape), gw, gs, gb, None, None, None


def pallas_fused_roi_step_epilogue(z_bmhw, delta_border_1mhw, w_eff_roi, s_eff_roi, b_roi,
                                   activate="tanh", has_border: bool = True):
    """kernels_pallas.py:663-690 (custom_vjp, nondiff (activate, has_border))."""
    a, slope = act_id(activate)
    return _Epilogue.apply(z_bmhw, delta_border_1mhw, w_eff_roi, s_eff_roi, b_roi, a, slope,
                           bool(has_border))


def fused_roi_step_epilogue(z_roi_bmhw, step_params, activate="tanh", norm: bool = True):
    """epilogue.py:28-56 (z already includes any border term)."""
    if not norm:
        raise NeurocellError("norm=False is not part of the MI355X path")
    M = z_roi_bmhw.shape[1]
    zero = torch.zeros(1, M, *z_roi_bmhw.shape[-2:], device=z_roi_bmhw.device)
    return pallas_fused_roi_step_epilogue(z_roi_bmhw, zero, step_params.w_eff_roi,
                                          step_params.s_eff_roi, step_params.b_roi, activate,
                                          False)


# ------------------------------------------------------------------ output port

class _Port(torch.autograd.Function):
    @staticmethod
    def forward(ctx, z, delta, pp, port_idx, fact, slope, has_border):
        z, pp = _f32(z), _f32(pp)
        B, M, h, wd = z.shape
        d = _f32(delta).reshape(M, h, wd) if has_border else None
        P = port_idx.numel()
        f = dict(device=z.device, dtype=torch.float32)
        out = torch.empty(B, P, **f)
        zo = torch.empty(B, M, P, **f)
        mean = torch.empty(B, M, **f)
        rstd = torch.empty(B, M, **f)
        pre = torch.empty(B, P, **f) if fact != 0 else None
        L = lib()
        ws = _ws(L.nc_epilogue_workspace_size(B, M, h, wd), z.device)
        call("nc_port_fwd", stream_ptr(), B, M, h, wd, int(has_border), fact, slope, P,
             ptr(port_idx), ptr(z), ptr(d), ptr(pp), ptr(out), ptr(zo), ptr(mean), ptr(rstd),
             ptr(pre), ptr(ws), ws.numel() * 4)
        ctx.save_for_backward(z, d if d is not None else z.new_empty(0), pp, port_idx, zo, mean,
                              rstd, pre if pre is not None else z.new_empty(0))
        ctx.args = (fact, slope, has_border, tuple(delta.shape))
        return out

    @staticmethod
    def backward(ctx, g_out):
        z, d, pp, port_idx, zo, mean, rstd, pre = ctx.saved_tensors
        fact, slope, hb, dshape = ctx.args
        B, M, h, wd = z.shape
        P = port_idx.numel()
        gz = torch.empty_like(z)
        gdb = torch.zeros(M, h, wd, device=z.device, dtype=torch.float32)
        gpp = torch.empty_like(pp)
        L = lib()
        ws = _ws(L.nc_epilogue_workspace_size(B, M, h, wd), z.device)
        call("nc_port_bwd", stream_ptr(), B, M, h, wd, int(hb), fact, slope, P, ptr(port_idx),
             ptr(z), ptr(d) if hb else None, ptr(pp), ptr(zo), ptr(mean), ptr(rstd),
             ptr(pre) if fact != 0 else None, ptr(_f32(g_out)), ptr(gz),
             ptr(gdb) if hb else None, ptr(gpp), 0, ptr(ws), ws.numel() * 4)
        return gz, gdb.reshape(dshape), gpp, None, None, None, None


def _port_idx(topology: ChipTopology2D, hw, device):
    rows, cols = topology.out_cells_roi()
    return torch.tensor((rows * hw[1] + cols).astype("int32"), device=device)


def pallas_fused_output_port_epilogue(z_roi_bmhw, delta_border_1mhw, step_params, topology,
                                      final_activate=None, has_border: bool = True):
    """kernels_pallas.py:1510-1551: returns (B, out_h, out_w); differentiable w.r.t. z, the
    border term and the port slices of ``step_params``."""
    fact, slope = act_id(final_activate)
    pp = torch.stack([step_params.w_eff_out.reshape(-1), step_params.s_eff_out.reshape(-1),
                      step_params.b_out.reshape(-1)])
    idx = _port_idx(topology, z_roi_bmhw.shape[-2:], z_roi_bmhw.device)
    out = _Port.apply(z_roi_bmhw, delta_border_1mhw, pp, idx, fact, slope, bool(has_border))
    oh, ow = topology.out_port.size
    return out.reshape(out.shape[0], oh, ow)


class _StdPort(torch.autograd.Function):
    @staticmethod
    def forward(ctx, z, delta, port_idx, has_border):
        z = _f32(z)
        B, M, h, wd = z.shape
        d = _f32(delta).reshape(M, h, wd) if has_border else None
        P = port_idx.numel()
        f = dict(device=z.device, dtype=torch.float32)
        zo = torch.empty(B, M, P, **f)
        mean = torch.empty(B, M, **f)
        rstd = torch.empty(B, M, **f)
        ws = _ws(lib().nc_epilogue_workspace_size(B, M, h, wd), z.device)
        call("nc_port_fwd", stream_ptr(), B, M, h, wd, int(has_border), 0, 0.0, P,
             ptr(port_idx), ptr(z), ptr(d), None, None, ptr(zo), ptr(mean), ptr(rstd), None,
             ptr(ws), ws.numel() * 4)
        ctx.save_for_backward(z, d if d is not None else z.new_empty(0), port_idx, zo, mean,
                              rstd)
        ctx.args = (has_border, tuple(delta.shape))
        return zo

    @staticmethod
    def backward(ctx, g_zo):
        z, d, port_idx, zo, mean, rstd = ctx.saved_tensors
        hb, dshape = ctx.args
        B, M, h, wd = z.shape
        P = port_idx.numel()
        gz = torch.empty_like(z)
        gdb = torch.zeros(M, h, wd, device=z.device, dtype=torch.float32)
        ws = _ws(lib().nc_epilogue_workspace_size(B, M, h, wd), z.device)
        call("nc_port_bwd", stream_ptr(), B, M, h, wd, int(hb), 0, 0.0, P, ptr(port_idx),
             ptr(z), ptr(d) if hb else None, None, ptr(zo), ptr(mean), ptr(rstd), None,
             ptr(_f32(g_zo)), ptr(gz), ptr(gdb) if hb else None, None, 0, ptr(ws),
             ws.numel() * 4)
        return gz, gdb.reshape(dshape), None, None


def pallas_standardize_output_port(z_bmhw, delta_border_1mhw, roi_out_offset=(16, 35),
                                   out_size=(8, 1), has_border: bool = True):
    """kernels_pallas.py:1256-1507: standardize(z + delta) at the output port only, as
    (B, M, out_h, out_w).  ``roi_out_offset`` is a (row, col) corner or, for a coordinate port,
    a (rows_tuple, cols_tuple) pair; cotangents (gz, gdb)."""
    B, M, h, w = z_bmhw.shape
    oh, ow = out_size
    if (isinstance(roi_out_offset, tuple) and len(roi_out_offset) == 2
            and isinstance(roi_out_offset[0], tuple)):
        rows = torch.tensor(roi_out_offset[0], dtype=torch.int64)
        cols = torch.tensor(roi_out_offset[1], dtype=torch.int64)
    else:
        r, c = roi_out_offset
        rr, cc = torch.meshgrid(torch.arange(oh) + int(r), torch.arange(ow) + int(c),
                                indexing="ij")
        rows, cols = rr.reshape(-1), cc.reshape(-1)
    if rows.numel() != oh * ow:
        raise ValueError("roi_out_offset does not match out_size")
    if (rows < 0).any() or (rows >= h).any() or (cols < 0).any() or (cols >= w).any():
        raise ValueError("output port lies outside the plane")
    idx = (rows * w + cols).to(torch.int32).to(z_bmhw.device)
    zo = _StdPort.apply(z_bmhw, delta_border_1mhw, idx, bool(has_border))
    return zo.reshape(B, M, oh, ow)


def fused_output_port_epilogue(z_roi_bmhw, step_params, topology, final_activate=None,
                               norm: bool = True):
    """epilogue.py:82-128 (z already includes any border term)."""
    if not norm:
        raise NeurocellError("norm=False is not part of the MI355X path")
    zero = torch.zeros(1, *z_roi_bmhw.shape[1:], device=z_roi_bmhw.device)
    return pallas_fused_output_port_epilogue(z_roi_bmhw, zero, step_params, topology,
                                             final_activate, False)


# ------------------------------------------------------------------ spectra

def _spec_ok(fft_shape):
    if not spectral_grid_supported(int(fft_shape[0]), int(fft_shape[1])):
        raise NeurocellError(f"spectral grid {tuple(fft_shape)} is not supported")


def precompute_filter_rfft2(filters_oihw, fft_shape=(64, 64)):
    """kernels_greens.py:240-259 (no gradient)."""
    _spec_ok(fft_shape)
    f = _f32(filters_oihw)
    M, _, kh, kw = f.shape
    out = torch.empty(M, fft_shape[0], fft_shape[1] // 2 + 1, device=f.device,
                      dtype=torch.complex64)
    call("nc_filter_spectrum_fwd", stream_ptr(), M, kh, kw, fft_shape[0], fft_shape[1], ptr(f),
         ptr(out))
    return out


def _filter_grad(g, kernel_size, shift, fft_shape, conj):
    """flip(crop(roll(irfft2(conj? conj(g) : g), shift))) -> (M, 1, Kh, Kw).  The spectrum is
    first reduced to what a real inverse transform keeps of it (the Hermitian parts of its DC
    and Nyquist columns), so any complex cotangent gives NumPy's / JAX's irfft2 result."""
    _spec_ok(fft_shape)
    g = g.contiguous()
    fh, fw = (int(v) for v in fft_shape)
    M = g.shape[0]
    kh, kw = kernel_size
    t = torch.empty_like(g)
    call("nc_spectrum_map", stream_ptr(), M, fh, fw, 0, 0, 1, 1.0, 1.0, int(conj), ptr(g),
         ptr(t))
    out = torch.empty(M, 1, kh, kw, device=g.device, dtype=torch.float32)
    call("nc_filter_spectrum_bwd", stream_ptr(), M, kh, kw, fh, fw, int(shift[0]) % fh,
         int(shift[1]) % fw, ptr(t), ptr(out), 0, 0)
    return out


def rfft2_unshifted_filter_grad_to_oihw(grad_ker_freq_unshifted_mhw, kernel_size=(23, 13),
                                        pad_hw=(11, 6), fft_shape=(64, 64), _torch_conj=False):
    """kernels_pallas.py:1558-1579: (M, Fh, Fw/2+1) complex cotangent -> (M, 1, Kh, Kw)."""
    return _filter_grad(grad_ker_freq_unshifted_mhw, kernel_size, pad_hw, fft_shape,
                        _torch_conj)


class _HoistNopad(torch.autograd.Function):
    @staticmethod
    def forward(ctx, filters, kernel_size, pad_hw, fft_shape, zero):
        ctx.args = (tuple(kernel_size), tuple(pad_hw), tuple(fft_shape))
        if zero:
            M = filters.shape[0]
            return torch.zeros(M, fft_shape[0], fft_shape[1] // 2 + 1, device=filters.device,
                               dtype=torch.complex64)
        return precompute_filter_rfft2(filters, fft_shape)

    @staticmethod
    def backward(ctx, g):
        ks, pad, fs = ctx.args
        return (rfft2_unshifted_filter_grad_to_oihw(g, ks, pad, fs, _torch_conj=True), None,
                None, None, None)


def hoist_filter_rfft2_nopad(filters_oihw, kernel_size=(23, 13), pad_hw=(11, 6),
                             fft_shape=(64, 64)):
    """kernels_pallas.py:1582-1604."""
    return _HoistNopad.apply(filters_oihw, kernel_size, pad_hw, fft_shape, False)


def hoist_filter_rfft2_zero_nopad(filters_oihw, kernel_size=(23, 13), pad_hw=(11, 6),
                                  fft_shape=(64, 64)):
    """kernels_pallas.py:1607-1631: zeros forward, unshifted filter-gradient backward."""
    return _HoistNopad.apply(filters_oihw, kernel_size, pad_hw, fft_shape, True)


class _PrunedConv(torch.autograd.Function):
    """conv2d_pruned_rfft_roi_step: z = irfft2(rfft2(x) * ker_freq) cropped at pad_hw;
    residuals (cell_freq, ker_freq); cotangents (g_cells, g_ker_freq_unshifted).  With
    ``shifted`` the ker_freq cotangent is conv2d_roi_rfft_step's (gz zero-padded to its window
    before the transform), the unshifted one times the phase of the pad."""

    @staticmethod
    def forward(ctx, x, ker_freq, roi_shape, pad_hw, fft_shape, need_dx, shifted=False):
        _spec_ok(fft_shape)
        x = _f32(x)
        kf = ker_freq.contiguous()
        B, hin, win = x.shape
        M = kf.shape[0]
        hout, wout = roi_shape
        z = torch.empty(B, M, hout, wout, device=x.device, dtype=torch.float32)
        xhat = torch.empty(B, fft_shape[0], fft_shape[1] // 2 + 1, device=x.device,
                           dtype=torch.complex64)
        call("nc_fftconv_fwd", stream_ptr(), B, M, hin, win, hout, wout, int(pad_hw[0]),
             int(pad_hw[1]), fft_shape[0], fft_shape[1], ptr(x), ptr(kf), ptr(z), ptr(xhat))
        ctx.save_for_backward(xhat, kf)
        ctx.args = (B, M, hin, win, hout, wout, tuple(pad_hw), tuple(fft_shape), bool(need_dx),
                    bool(shifted))
        return z

    @staticmethod
    def backward(ctx, gz):
        xhat, kf = ctx.saved_tensors
        B, M, hin, win, hout, wout, pad, fs, need_dx, shifted = ctx.args
        dev = xhat.device
        dx = torch.zeros(B, hin, win, device=dev, dtype=torch.float32)
        dkf = torch.empty_like(kf)
        L = lib()
        ws = _ws(L.nc_fftconv_bwd_workspace_size(B, M, fs[0], fs[1]), dev)
        call("nc_fftconv_bwd", stream_ptr(), B, M, hin, win, hout, wout, pad[0], pad[1], fs[0],
             fs[1], ptr(_f32(gz)), ptr(xhat), ptr(kf), int(need_dx),
             ptr(dx) if need_dx else None, ptr(dkf), 0, 1, ptr(ws), ws.numel() * 4)
        if shifted:
            # rfft2(pad(gz)) = rfft2(gz) * W^(k.pad); in the conjugate (autograd) convention
            # the cotangent takes the conjugate phase, W^(-k.pad)
            call("nc_spectrum_map", stream_ptr(), M, fs[0], fs[1], (-pad[0]) % fs[0],
                 (-pad[1]) % fs[1], 0, 1.0, 1.0, 0, ptr(dkf), ptr(dkf))
        return dx, dkf, None, None, None, None, None


def conv2d_pruned_rfft_roi_step(roi_cells_bhw, ker_freq_mhw, roi_shape=(40, 50), pad_hw=(11, 6),
                                fft_shape=(64, 64), need_dx: bool = True):
    """kernels_pallas.py:1759-1826."""
    return _PrunedConv.apply(roi_cells_bhw, ker_freq_mhw, tuple(roi_shape), tuple(pad_hw),
                             tuple(fft_shape), bool(need_dx))


class _Hybrid(torch.autograd.Function):
    """conv2d_hybrid_nopad_roi_step: the forward correlates with the filters' spectrum; the
    cotangents are (g_cells, zeros for the stop-gradient filters, the unshifted spectral
    cotangent for the token)."""

    @staticmethod
    def forward(ctx, x, filters, token, pad_hw, fft_shape, need_dx):
        kf = precompute_filter_rfft2(filters, fft_shape)
        h, w = x.shape[-2:]
        ctx.inner = _PrunedConv
        z = _PrunedConv.forward(ctx, x, kf, (h, w), pad_hw, fft_shape, need_dx)
        return z

    @staticmethod
    def backward(ctx, gz):
        dx, dkf, *_ = _PrunedConv.backward(ctx, gz)
        return dx, None, dkf, None, None, None


def conv2d_hybrid_nopad_roi_step(roi_cells_bhw, filters_oihw, ker_freq_token, pad_hw=(11, 6),
                                 fft_shape=(64, 64), need_dx: bool = True):
    """kernels_pallas.py:1634-1697: forward on the filters, filter gradient through the token
    (``hoist_filter_rfft2_zero_nopad``)'s unshifted cotangent.  On MI355X the forward is the
    same spectral correlation as every other backend."""
    return _Hybrid.apply(roi_cells_bhw, filters_oihw.detach(), ker_freq_token, tuple(pad_hw),
                         tuple(fft_shape), bool(need_dx))


def conv2d_small_kernel_roi_step(roi_cells_bhw, filters_oihw, pad_hw=(1, 1),
                                 need_dx: bool = True):
    """kernels_pallas.py:1700-1756: SAME-ROI correlation with (dx, dG) cotangents."""
    h, w = roi_cells_bhw.shape[-2:]
    kh, kw = filters_oihw.shape[-2:]
    fs = (_npow2(h + kh - 1), _npow2(w + kw - 1))
    kf = hoist_filter_rfft2_nopad(filters_oihw, (kh, kw), tuple(pad_hw), fs)
    return _PrunedConv.apply(roi_cells_bhw, kf, (h, w), tuple(pad_hw), fs, bool(need_dx))


def conv2d_batched_nchw(cells_nchw, filters_oihw, padding="VALID", **unused):
    """kernels_greens.py:177-217 for C_in = 1, stride 1: VALID or SAME correlation."""
    if cells_nchw.shape[1] != 1 or unused.get("feature_group_count", 1) != 1:
        raise NeurocellError("conv2d_batched_nchw supports C_in = 1, ungrouped")
    x = cells_nchw[:, 0]
    H, W = x.shape[-2:]
    kh, kw = filters_oihw.shape[-2:]
    if padding == "VALID":
        fs = (_npow2(H), _npow2(W))
        kf = hoist_filter_rfft2_nopad(filters_oihw, (kh, kw), (kh - 1, kw - 1), fs)
        return _PrunedConv.apply(x, kf, (H - kh + 1, W - kw + 1), (kh - 1, kw - 1), fs, True)
    if padding == "SAME":
        return conv2d_small_kernel_roi_step(x, filters_oihw, ((kh - 1) // 2, (kw - 1) // 2))
    raise NeurocellError(f"padding {padding!r} is not supported")


# ------------------------------------------------------------------ kernels_greens.py operators

def _planes(shape):
    n = 1
    for v in shape:
        n *= int(v)
    return n


def _grid_for(h: int, w: int):
    """The smallest supported spectral grid holding an h x w linear correlation support."""
    gh, gw = max(16, _npow2(h)), max(16, _npow2(w))
    if gh <= 64 and gw <= 64:
        return gh, gw
    gh, gw = max(64, gh), max(64, gw)
    if gh > 256 or gw > 256:
        raise NeurocellError(f"a {h}x{w} correlation support exceeds the 256x256 grid")
    return gh, gw


class _Rfft2(torch.autograd.Function):
    """rfft2_pruned: half-spectra of the real planes zero-padded to the grid.  Its adjoint
    (the autograd convention, dL/dRe + i dL/dIm) is Re sum over the half-spectrum of
    g e^{+i theta}: N * irfft2 of g with the interior columns halved (and the edge columns'
    Hermitian parts, which is all a real inverse keeps of them)."""

    @staticmethod
    def forward(ctx, x, fft_shape):
        _spec_ok(fft_shape)
        x = _f32(x)
        fh, fw = (int(v) for v in fft_shape)
        h, w = x.shape[-2:]
        n = _planes(x.shape[:-2])
        out = torch.empty(*x.shape[:-2], fh, fw // 2 + 1, device=x.device,
                          dtype=torch.complex64)
        call("nc_plane_spectrum", stream_ptr(), n, h, w, fh, fw, 0, 0, ptr(x), ptr(out))
        ctx.args = (tuple(x.shape), (fh, fw))
        return out

    @staticmethod
    def backward(ctx, g):
        shape, (fh, fw) = ctx.args
        n, N = _planes(shape[:-2]), float(fh * fw)
        g = g.contiguous()
        t = torch.empty_like(g)
        call("nc_spectrum_map", stream_ptr(), n, fh, fw, 0, 0, 1, N, 0.5 * N, 0, ptr(g), ptr(t))
        gx = torch.empty(shape, device=g.device, dtype=torch.float32)
        ws = _ws(lib().nc_irfft2_pruned_workspace_size(n, fh, fw), g.device)
        call("nc_irfft2_pruned", stream_ptr(), n, shape[-2], shape[-1], 0, 0, fh, fw, ptr(t),
             ptr(gx), ptr(ws), ws.numel() * 4)
        return gx, None


def rfft2_pruned(x, fft_shape=(64, 64)):
    """kernels_greens.py:25-44: rfft2 of the (..., H_in, W_in) planes zero-padded to
    ``fft_shape`` (H_in <= Fh, W_in <= Fw), as (..., Fh, Fw/2+1) complex64; differentiable."""
    return _Rfft2.apply(x, tuple(fft_shape))


class _Irfft2(torch.autograd.Function):
    """irfft2_pruned; its adjoint is (c_k / N) rfft2 of the cotangent placed at the window,
    c_k = 1 on the DC and Nyquist columns and 2 elsewhere."""

    @staticmethod
    def forward(ctx, xf, roi_shape, pad_hw, fft_shape):
        _spec_ok(fft_shape)
        if xf.dtype != torch.complex64 or not xf.is_cuda:
            raise NeurocellError("expected a complex64 device tensor")
        xf = xf.contiguous()
        fh, fw = (int(v) for v in fft_shape)
        if tuple(xf.shape[-2:]) != (fh, fw // 2 + 1):
            raise NeurocellError(f"spectrum shape {tuple(xf.shape[-2:])} does not match the "
                                 f"grid {fh}x{fw}")
        rh, rw = (int(v) for v in roi_shape)
        ph, pw = (int(v) for v in pad_hw)
        n = _planes(xf.shape[:-2])
        out = torch.empty(*xf.shape[:-2], rh, rw, device=xf.device, dtype=torch.float32)
        ws = _ws(lib().nc_irfft2_pruned_workspace_size(n, fh, fw), xf.device)
        call("nc_irfft2_pruned", stream_ptr(), n, rh, rw, ph, pw, fh, fw, ptr(xf), ptr(out),
             ptr(ws), ws.numel() * 4)
        ctx.args = (tuple(xf.shape[:-2]), (rh, rw), (ph, pw), (fh, fw))
        return out

    @staticmethod
    def backward(ctx, g):
        lead, (rh, rw), (ph, pw), (fh, fw) = ctx.args
        n, N = _planes(lead), float(fh * fw)
        gx = torch.empty(*lead, fh, fw // 2 + 1, device=g.device, dtype=torch.complex64)
        call("nc_plane_spectrum", stream_ptr(), n, rh, rw, fh, fw, ph, pw, ptr(_f32(g)),
             ptr(gx))
        call("nc_spectrum_map", stream_ptr(), n, fh, fw, 0, 0, 0, 1.0 / N, 2.0 / N, 0, ptr(gx),
             ptr(gx))
        return gx, None, None, None


def irfft2_pruned(x_freq, roi_shape, pad_hw, fft_shape=(64, 64)):
    """kernels_greens.py:47-66: irfft2 on ``fft_shape`` sliced to
    [..., r_h : r_h + roi_h, r_w : r_w + roi_w]; differentiable."""
    return _Irfft2.apply(x_freq, tuple(roi_shape), tuple(pad_hw), tuple(fft_shape))


def _select_batch_groups(batch_size: int, max_groups: int = 8) -> int:
    """kernels_greens.py:69-81 (kept for API compatibility: the MI355X filter gradient sums
    every sample in one fixed-order frequency-domain reduction, so no grouping is needed)."""
    eff = min(batch_size, max_groups)
    if batch_size >= 16:
        eff = min(eff, max(1, batch_size // 16))
    for g in range(eff, 0, -1):
        if batch_size % g == 0:
            return g
    return 1


def conv2d_grouped_filter_grad(roi_cells_bhw, g_z_roi, pad_hw, max_groups: int = 8):
    """kernels_greens.py:84-123: the filter gradient dG (M, 1, Kh, Kw) of
    conv2d(roi_cells[:, None], filters, padding=((r_h, r_h), (r_w, r_w))) for the output
    cotangent g_z_roi (B, M, h_out, w_out), Kh = h_in + 2 r_h - h_out + 1.  Here the batch sum
    runs in the frequency domain (unshifted Plancherel, nc_fftconv_bwd without dx) and one
    inverse per direction realigns it (nc_filter_spectrum_bwd, roll Kh - 1 - r_h);
    ``max_groups`` is accepted and has no effect on the result."""
    x, gz = _f32(roi_cells_bhw), _f32(g_z_roi)
    B, hin, win = x.shape
    Bz, M, hout, wout = gz.shape
    if Bz != B:
        raise ValueError("batch sizes of the cells and the cotangent differ")
    rh, rw = (int(v) for v in pad_hw)
    kh, kw = hin + 2 * rh - hout + 1, win + 2 * rw - wout + 1
    if kh <= 0 or kw <= 0 or rh < 0 or rw < 0:
        raise ValueError("inconsistent shapes for the filter gradient")
    fh, fw = _grid_for(max(hin + rh, hout, kh), max(win + rw, wout, kw))
    F = fh * (fw // 2 + 1)
    dev = x.device
    xhat = torch.empty(B, F, device=dev, dtype=torch.complex64)
    call("nc_plane_spectrum", stream_ptr(), B, hin, win, fh, fw, 0, 0, ptr(x), ptr(xhat))
    ghat = torch.zeros(M, F, device=dev, dtype=torch.complex64)  # unused without dx
    dgh = torch.empty(M, F, device=dev, dtype=torch.complex64)
    ws = _ws(lib().nc_fftconv_bwd_workspace_size(B, M, fh, fw), dev)
    call("nc_fftconv_bwd", stream_ptr(), B, M, hin, win, hout, wout, 0, 0, fh, fw, ptr(gz),
         ptr(xhat), ptr(ghat), 0, None, ptr(dgh), 0, 0, ptr(ws), ws.numel() * 4)
    out = torch.empty(M, 1, kh, kw, device=dev, dtype=torch.float32)
    call("nc_filter_spectrum_bwd", stream_ptr(), M, kh, kw, fh, fw, (kh - 1 - rh) % fh,
         (kw - 1 - rw) % fw, ptr(dgh), ptr(out), 0, 0)
    return out


def rfft2_filter_grad_to_oihw(grad_ker_freq_mhw, kernel_size=(23, 13), fft_shape=(64, 64)):
    """kernels_greens.py:262-275: irfft2 of the (M, Fh, Fw/2+1) frequency cotangent, cropped
    to (Kh, Kw) and flipped -> (M, 1, Kh, Kw) (no roll: the shifted convention)."""
    return _filter_grad(grad_ker_freq_mhw, kernel_size, (0, 0), fft_shape, False)


def hoist_filter_rfft2(filters_oihw, kernel_size=(23, 13), fft_shape=(64, 64)):
    """kernels_greens.py:278-313: precompute_filter_rfft2 whose backward turns the shifted
    frequency cotangent into OIHW filter gradients (rfft2_filter_grad_to_oihw)."""
    return _HoistNopad.apply(filters_oihw, tuple(kernel_size), (0, 0), tuple(fft_shape), False)


def hoist_filter_rfft2_zero_fwd(filters_oihw, kernel_size=(23, 13), fft_shape=(64, 64)):
    """kernels_greens.py:428-465: zeros forward, rfft2_filter_grad_to_oihw backward."""
    return _HoistNopad.apply(filters_oihw, tuple(kernel_size), (0, 0), tuple(fft_shape), True)


def conv2d_roi_rfft_step(roi_cells_bhw, ker_freq_mhw, roi_shape=(40, 50), pad_hw=(11, 6),
                         fft_shape=(64, 64), need_dx: bool = True):
    """kernels_greens.py:316-400: the SAME ROI correlation of the cells with the hoisted filter
    spectra; residuals (cell_freq, ker_freq); cotangents (g_cells, g_ker_freq) with the
    reference's shifted ker_freq cotangent (gz zero-padded at pad_hw before its transform)."""
    return _PrunedConv.apply(roi_cells_bhw, ker_freq_mhw, tuple(roi_shape), tuple(pad_hw),
                             tuple(fft_shape), bool(need_dx), True)


def conv2d_valid_rfft_precomputed(cells_bhw, ker_freq_mhw, roi_shape=(40, 50),
                                  kernel_size=(23, 13), fft_shape=(64, 64)):
    """kernels_greens.py:403-425: the VALID correlation of the full (B, H, W) grid read at
    offset (Kh - 1, Kw - 1)."""
    kh, kw = kernel_size
    return conv2d_roi_rfft_step(cells_bhw, ker_freq_mhw, roi_shape, (kh - 1, kw - 1),
                                fft_shape, True)


class _HybridRoi(torch.autograd.Function):
    """conv2d_hybrid_roi_step: forward on the filters (the reference's direct conv; here the
    same spectral correlation), cotangents (g_cells, zeros for the filters, the shifted
    spectral cotangent for the token)."""

    @staticmethod
    def forward(ctx, x, filters, token, pad_hw, fft_shape, need_dx):
        kf = precompute_filter_rfft2(filters, fft_shape)
        h, w = x.shape[-2:]
        ctx.fshape = tuple(filters.shape)
        return _PrunedConv.forward(ctx, x, kf, (h, w), pad_hw, fft_shape, need_dx, True)

    @staticmethod
    def backward(ctx, gz):
        dx, dkf, *_ = _PrunedConv.backward(ctx, gz)
        gf = torch.zeros(ctx.fshape, device=dx.device, dtype=torch.float32)
        return dx, gf, dkf, None, None, None


def conv2d_hybrid_roi_step(roi_cells_bhw, filters_oihw, ker_freq_token, pad_hw=(11, 6),
                           fft_shape=(64, 64), need_dx: bool = True):
    """kernels_greens.py:468-551 with ``hoist_filter_rfft2_zero_fwd``'s token.  The reference's
    rule pairs a direct conv padded by pad_hw with a spectral cotangent shifted by pad_hw, which
    agree only for SAME pads (2 r = K - 1); other pads raise."""
    kh, kw = filters_oihw.shape[-2:]
    if 2 * int(pad_hw[0]) != kh - 1 or 2 * int(pad_hw[1]) != kw - 1:
        raise NeurocellError("conv2d_hybrid_roi_step takes SAME pads ((Kh-1)/2, (Kw-1)/2)")
    return _HybridRoi.apply(roi_cells_bhw, filters_oihw, ker_freq_token, tuple(pad_hw),
                            tuple(fft_shape), bool(need_dx))


# ------------------------------------------------------------------ epilogue.py operators

class _Standardize(torch.autograd.Function):
    @staticmethod
    def forward(ctx, z):
        z = _f32(z)
        n = z.shape[-1] * z.shape[-2]
        planes = _planes(z.shape[:-2])
        out = torch.empty_like(z)
        mean = torch.empty(planes, device=z.device, dtype=torch.float32)
        rstd = torch.empty_like(mean)
        call("nc_standardize_fwd", stream_ptr(), planes, n, ptr(z), ptr(out), ptr(mean),
             ptr(rstd))
        ctx.save_for_backward(z, mean, rstd)
        return out

    @staticmethod
    def backward(ctx, g):
        z, mean, rstd = ctx.saved_tensors
        gx = torch.empty_like(z)
        call("nc_standardize_bwd", stream_ptr(), mean.numel(), z.shape[-1] * z.shape[-2], ptr(z),
             ptr(mean), ptr(rstd), ptr(_f32(g)), ptr(gx))
        return gx


def standardize_spatial_nchw(z_bmhw):
    """epilogue.py:20-25: each (b, m) plane standardised to zero mean and unit variance
    (population variance, eps 1e-5); differentiable."""
    return _Standardize.apply(z_bmhw)


def fused_roi_epilogue(z_roi_bmhw, step_params, c_border_bhw, topology, activate="tanh",
                       norm: bool = True):
    """epilogue.py:59-79: the ROI update of ``fused_roi_step_epilogue`` embedded into the
    full-grid border template (B, H, W) at the ROI; differentiable w.r.t. z, the step
    parameters and the template's border cells."""
    roi_next = fused_roi_step_epilogue(z_roi_bmhw, step_params, activate, norm)
    rh, rw = topology.pad_h, topology.pad_w
    H, W = topology.grid_shape
    out = c_border_bhw.clone()
    out[:, rh:H - rh, rw:W - rw] = roi_next
    return out

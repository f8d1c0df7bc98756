"""Propagation entry point: ``propagate_vnn_2d`` (propagator.py:209-734) on the gfx950 path.

Every accepted ``backend`` string routes to the single MI355X implementation (the step
executor in ``engine.py``: spectral correlation + fused epilogues), so the name set and its
validation are kept for API compatibility (propagator.py:58-65, 231-234).  The whole d-step
forward is one autograd node whose backward is the executor's reverse pass (the chain of
the reference's custom VJPs), giving gradients w.r.t. ``params.cell_params`` and
``params.greens_filters``.
"""
from __future__ import annotations

from collections import OrderedDict

import numpy as np
import torch

from ._lib import NeurocellError
from .engine import StepPlan, flatten_inputs, inv_tau_f32, port_input_shapes
from .topology import ChipTopology2D, CoordinatePortSpec

SUPPORTED_BACKENDS = ("auto", "nchw_direct", "rfft_hoisted", "nchw_rfft_bwd", "pallas_fused",
                      "pallas_sram")


def select_optimal_backend(topology: ChipTopology2D) -> str:
    """propagator.py:68-85 cost model, kept for API compatibility: on MI355X every backend
    string runs the same spectral + fused-epilogue path, whose grid the topology fixes."""
    kh, kw = topology.kernel_size
    roi_h, roi_w = topology.roi_shape
    if roi_h * roi_w < 256:
        return "nchw_direct"
    fh, fw = topology.fft_shape
    fits = (roi_h + kh - 1 <= fh) and (roi_w + kw - 1 <= fw)
    if topology.padding_mode != "CIRCULAR" and kh * kw > 512 and fits:
        return "pallas_sram"
    return "pallas_fused"


def cropped_bbox(spatial_mask, topology: ChipTopology2D):
    """The sub-ROI a spatial mask selects (propagator.py:235-241): its ``roi_bbox``, or None
    without a mask, for a full-ROI mask, and in CIRCULAR mode (the reference ignores the
    crop there and runs the whole grid)."""
    if (spatial_mask is None or spatial_mask.is_full_roi
            or topology.padding_mode == "CIRCULAR"):
        return None
    return tuple(int(v) for v in spatial_mask.roi_bbox)


class _PlanCache:
    """Static launch plans per (topology, B, sub-ROI, port shapes, activations), least
    recently used first out.  A plan holds its bucket's whole activation set in HBM, so the
    cache keeps at most ``capacity`` of them; topologies compare by value."""

    def __init__(self, capacity: int = 16):
        self.plans = OrderedDict()
        self.capacity = int(capacity)

    def get(self, topology, B, port_shapes, roi_bbox, activate, final_activate, hard_pin_io,
            training, device, gated_filters=False, sharpen=None, universe=False):
        sk = None if sharpen is None else np.asarray(sharpen, np.float32)
        key = (topology, B, tuple(port_shapes), roi_bbox, str(activate),
               str(final_activate), bool(hard_pin_io), bool(training), str(device),
               bool(gated_filters), None if sk is None else (sk.shape, sk.tobytes()),
               bool(universe))
        p = self.plans.get(key)
        if p is None:
            p = self.plans[key] = StepPlan(topology, B, port_shapes, roi_bbox=roi_bbox,
                                           activate=activate, final_activate=final_activate,
                                           hard_pin_io=hard_pin_io, training=training,
                                           device=device, gated_filters=gated_filters,
                                           sharpen=sk, universe=universe)
            while len(self.plans) > self.capacity:
                self.plans.popitem(last=False)
        else:
            self.plans.move_to_end(key)
        return p


_PLANS = _PlanCache()


class _Propagate(torch.autograd.Function):
    """The d-step forward as one node: outputs the port predictions, and the final universe
    too when the plan was built with ``return_universe``."""

    @staticmethod
    def forward(ctx, cell, filt, x_flat, plan, codd, need_grad, return_universe):
        mode, it, thr = codd
        cell, filt = cell.contiguous(), filt.contiguous()
        # each call owns its activations so several graphs can be alive at once
        run = plan.fresh() if need_grad else plan
        out = run.forward(cell, filt, x_flat, codd_mode=mode, inv_tau=it,
                          active_threshold=thr).clone()
        ctx.run, ctx.codd = run, codd
        ctx.save_for_backward(cell, filt)
        ctx.set_materialize_grads(False)
        if return_universe:
            return out, run.univ.clone()
        return out

    @staticmethod
    def backward(ctx, g_out, g_univ=None):
        cell, filt = ctx.saved_tensors
        mode, it, thr = ctx.codd
        run = ctx.run
        g_cell = torch.empty_like(cell)
        g_filt = torch.empty_like(filt)
        if g_out is None and not run.universe:
            g_out = torch.zeros_like(run.out)
        c = lambda t: None if t is None else t.contiguous()
        run.backward(cell, filt, c(g_out), g_cell, g_filt, codd_mode=mode, inv_tau=it,
                     active_threshold=thr, g_universe=c(g_univ))
        ctx.run = None
        return g_cell, g_filt, None, None, None, None, None


def _host_kernel(k):
    """A sharpening stencil (array-like or tensor) as a float32 host array, or None."""
    if k is None:
        return None
    if isinstance(k, torch.Tensor):
        k = k.detach().cpu().numpy()
    return np.asarray(k, np.float32)


def propagate_vnn_2d(params, inputs, topology: ChipTopology2D, activate="tanh",
                     final_activate=None, norm: bool = True, sharpen_filter=None,
                     gated_filters: bool = False, hard_pin_io: bool = False,
                     backend: str = "nchw_direct", return_universe: bool = False,
                     spatial_mask=None, codd_mode: str = "continuous",
                     state_temperature: float = 1.0, active_threshold: float = 0.6):
    """propagator.py:209-734: (B, out_h, out_w) port predictions, differentiable w.r.t. the
    VNNParams leaves.  ``spatial_mask`` (an AdaptiveMaskSpec) runs on its cropped sub-ROI.
    With ``return_universe`` also the final (B, H, W) universe (propagator.py:684-734), also
    differentiable; an output port outside the ROI is read from that universe as well."""
    if backend not in SUPPORTED_BACKENDS:
        raise ValueError(f"Unsupported backend '{backend}'; choose from {SUPPORTED_BACKENDS}.")
    from .params import SUPPORTED_CODD_MODES
    if codd_mode not in SUPPORTED_CODD_MODES:
        raise ValueError(f"Unsupported codd_mode '{codd_mode}'; choose from "
                         f"{SUPPORTED_CODD_MODES}.")
    if not norm:
        raise NeurocellError("norm=False is not part of the MI355X path")
    roi_bbox = cropped_bbox(spatial_mask, topology)
    x_flat = flatten_inputs(inputs, topology)
    cell, filt = params.cell_params, params.greens_filters
    need_grad = torch.is_grad_enabled() and (cell.requires_grad or filt.requires_grad)
    plan = _PLANS.get(topology, x_flat.shape[0], port_input_shapes(inputs, topology), roi_bbox,
                      activate, final_activate, hard_pin_io, need_grad, cell.device,
                      gated_filters, _host_kernel(sharpen_filter), bool(return_universe))
    codd = (codd_mode, inv_tau_f32(float(state_temperature)), float(active_threshold))
    res = _Propagate.apply(cell, filt, x_flat, plan, codd, need_grad, bool(return_universe))
    oh, ow = topology.out_port.size
    if return_universe:
        out, univ = res
        return out.reshape(out.shape[0], oh, ow), univ
    return res.reshape(res.shape[0], oh, ow)


def inject_inputs_roi_2d(inputs, topology: ChipTopology2D, dtype=torch.float32, roi_bbox=None):
    """propagator.py:135-191: (roi_cells, True) when every port fits the (cropped) ROI, else
    (None, False).  Runs the executor's gather kernel."""
    from ._lib import call, ptr, stream_ptr
    x_flat = flatten_inputs(inputs, topology)
    plan = _PLANS.get(topology, x_flat.shape[0], port_input_shapes(inputs, topology), roi_bbox,
                      "tanh", None, False, False, x_flat.device)
    if plan.t0_grid:
        return None, False
    roi = torch.empty(x_flat.shape[0], plan.h, plan.w, device=x_flat.device, dtype=dtype)
    call("nc_inject_roi", stream_ptr(), x_flat.shape[0], plan.n_in, ptr(x_flat), plan.h * plan.w,
         ptr(plan.src), ptr(roi))
    return roi, True


_GRID_MAPS = OrderedDict()


def _grid_inject_map(topology: ChipTopology2D, port_shapes, device):
    """Gather map (H*W,) of the full-grid injection: for each grid cell the index of the
    flattened input written there, or -1.  Later ports overwrite earlier ones at a shared
    cell, as the reference's successive ``.at[].set`` do."""
    key = (topology, tuple(port_shapes), str(device))
    m = _GRID_MAPS.get(key)
    if m is not None:
        _GRID_MAPS.move_to_end(key)
        return m
    H, W = topology.grid_shape
    src = np.full(H * W, -1, np.int32)
    e = 0
    for port, (ih, iw) in zip(topology.in_ports, port_shapes):
        if isinstance(port, CoordinatePortSpec):
            for k, (r, c) in enumerate(port.coords):
                src[r * W + c] = e + k
            e += port.num_points
            continue
        r0, c0 = port.offset
        if r0 < 0 or c0 < 0 or r0 + ih > H or c0 + iw > W:
            raise ValueError(f"input port {port.name!r} of {ih}x{iw} at {port.offset} lies "
                             "outside the grid")
        for i in range(ih):
            src[(r0 + i) * W + c0:(r0 + i) * W + c0 + iw] = e + i * iw + np.arange(iw)
        e += ih * iw
    m = _GRID_MAPS[key] = (torch.tensor(src, device=device), e)
    while len(_GRID_MAPS) > 32:
        _GRID_MAPS.popitem(last=False)
    return m


def inject_inputs_2d(inputs, topology: ChipTopology2D, dtype=torch.float32):
    """propagator.py:103-132: the batched port inputs written into a zero (B, H, W) field
    (rectangular ports at their offsets - a 3-D per-port input with its own (ih, iw) -
    coordinate ports at their cells).  Runs the executor's gather kernel over the grid."""
    from ._lib import call, ptr, stream_ptr
    if dtype != torch.float32:
        raise NeurocellError("the MI355X path injects float32 fields")
    x_flat = flatten_inputs(inputs, topology)
    src, n_in = _grid_inject_map(topology, port_input_shapes(inputs, topology), x_flat.device)
    if n_in != x_flat.shape[1]:
        raise NeurocellError(f"inputs carry {x_flat.shape[1]} values per sample, the ports "
                             f"take {n_in}")
    H, W = topology.grid_shape
    cells = torch.empty(x_flat.shape[0], H, W, device=x_flat.device, dtype=dtype)
    call("nc_inject_roi", stream_ptr(), x_flat.shape[0], n_in, ptr(x_flat), H * W, ptr(src),
         ptr(cells))
    return cells

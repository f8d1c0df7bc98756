"""Parameter PyTree and the pre-step factored Codd fusion.

Mirror of the reference's ``neurocell/params.py``: ``VNNParams`` (:83-113) packs
``[W, B, S_raw]`` as one contiguous ``(3, H, W)`` tensor plus ``(M, 1, Kh, Kw)`` OIHW Green's
filters; ``compute_codd_state_probs`` (:31-80) and ``precompute_step_params`` (:220-322)
keep their signatures and are differentiable (torch autograd), computed by the gfx950
Codd-fusion kernels (``nc_codd_fuse_fwd``/``_bwd``).
"""
from __future__ import annotations

from typing import NamedTuple

import numpy as np
import torch

from . import _abi
from ._lib import NeurocellError, call, ptr, stream_ptr
from .engine import act_id, inv_tau_f32
from .topology import ChipTopology2D

STATE_ACTIVE = 0.7
STATE_SIGNAL = 0.2
STATE_ACTIVE_VALUE = 1.0
STATE_SIGNAL_VALUE = 0.0

SUPPORTED_CODD_MODES = ("continuous", "annealed", "ste_binary", "ste_ternary")


class VNNParams(NamedTuple):
    """Learnable parameters (params.py:83-113): cell_params (3,H,W) = [W, B, S_raw] and
    greens_filters (M,1,Kh,Kw) OIHW."""
    cell_params: torch.Tensor
    greens_filters: torch.Tensor

    @property
    def weights(self):
        return self.cell_params[0]

    @property
    def biases(self):
        return self.cell_params[1]

    @property
    def states(self):
        return self.cell_params[2]

    @property
    def filters_ihwo(self):
        """Green's filters in the legacy (1, Kh, Kw, M) layout."""
        return self.greens_filters.permute(1, 2, 3, 0)


class PrecomputedStepParams(NamedTuple):
    """Pre-step fused parameters (params.py:116-135).  ``border_patch`` is the hoisted
    border template with the ROI zeroed, already cut to the (cropped) ROI's receptive field;
    ``port_params`` stacks (w_eff_out, s_eff_out, b_out) over the output cells."""
    w_eff_roi: torch.Tensor
    s_eff_roi: torch.Tensor
    b_roi: torch.Tensor
    border_2d: torch.Tensor
    w_eff_out: torch.Tensor
    s_eff_out: torch.Tensor
    b_out: torch.Tensor
    w_pinned: torch.Tensor
    b_full: torch.Tensor
    s_prob: torch.Tensor
    border_patch: torch.Tensor = None
    port_params: torch.Tensor = None


def _variance_scaling_trunc(shape, scale, fan_in, gen):
    """variance_scaling(scale, "fan_in", "truncated_normal"): a unit normal truncated to
    [-2, 2], times sqrt(scale / fan_in) / 0.87962566103423978 (the truncated unit normal's
    standard deviation), drawn on the host from ``gen``."""
    t = torch.empty(shape, dtype=torch.float32)
    torch.nn.init.trunc_normal_(t, 0.0, 1.0, -2.0, 2.0, generator=gen)
    return t * float(np.sqrt(scale / fan_in) / 0.87962566103423978)


def init_vnn_params(rng, topology: ChipTopology2D, dtype=torch.float32,
                    clear_outside_io: bool = False, legacy_compat: bool = True,
                    device=None) -> VNNParams:
    """params.py:145-217 with a torch generator: states sigmoid(trunc-normal), weights
    trunc-normal (scale 1/sqrt(depth*N), fan-in H), biases zero, filters drawn as (1,Kh,Kw,M)
    (scale 1/sqrt(Kh*Kw*M), fan-in Kh*Kw) then laid out OIHW; IO cells pinned to 1.  ``rng`` is
    an int seed or a ``torch.Generator``.  The draws follow the reference's distributions and
    key order (states, weights, filters) but not JAX's threefry bit stream."""
    if dtype != torch.float32:
        raise NeurocellError("the MI355X path computes in float32")
    gen = rng if isinstance(rng, torch.Generator) else torch.Generator().manual_seed(int(rng))
    H, W = topology.grid_shape
    kh, kw = topology.kernel_size
    M = topology.directions
    init_scale = 1.0 / np.sqrt(topology.depth * topology.N)
    filt_scale = 1.0 / np.sqrt(kh * kw * M)
    states = torch.sigmoid(_variance_scaling_trunc((H, W), init_scale, H, gen))
    weights = _variance_scaling_trunc((H, W), init_scale, H, gen)
    filters_ihwo = _variance_scaling_trunc((1, kh, kw, M), filt_scale, kh * kw, gen)
    if clear_outside_io:
        for port in topology.in_ports:
            c0 = port.offset[1]
            states[:, : c0 + 1] = 0.0
            weights[:, : c0 + 1] = 0.0
        out_c = topology.out_port.offset[1]
        states[:, out_c:] = 0.0
        weights[:, out_c:] = 0.0
    io = torch.as_tensor(np.asarray(topology.io_state_mask, dtype=bool))
    states = torch.where(io, torch.tensor(STATE_ACTIVE_VALUE), states)
    weights = torch.where(io, torch.tensor(1.0), weights)
    cell = torch.stack([weights, torch.zeros(H, W), states])
    filt = filters_ihwo.permute(3, 0, 1, 2).contiguous()
    if device is None:
        from ._lib import require_device
        device = require_device()
    return VNNParams(cell.to(device), filt.to(device))


def _check_mode(codd_mode):
    if codd_mode not in SUPPORTED_CODD_MODES:
        raise ValueError(f"Unsupported codd_mode '{codd_mode}'; choose from "
                         f"{SUPPORTED_CODD_MODES}.")


class _Geometry:
    """Device-side static operands of the Codd fusion for one topology and sub-ROI."""

    _cache: dict = {}

    def __init__(self, topology: ChipTopology2D, roi_bbox, device):
        H, W = topology.grid_shape
        kh, kw = topology.kernel_size
        roi_h, roi_w = topology.roi_shape
        r0, r1, c0, c1 = roi_bbox if roi_bbox is not None else (0, roi_h, 0, roi_w)
        self.chip = _abi.ChipDesc(H, W, kh, kw, topology.directions, topology.pad_h,
                                  topology.pad_w, roi_h, roi_w, r0, r1, c0, c1)
        self.h, self.w = r1 - r0, c1 - c0
        self.Hp, self.Wp = self.h + kh - 1, self.w + kw - 1
        rows, cols = topology.out_cells_roi()
        self.P = int(rows.size)
        self.out_size = tuple(topology.out_port.size)
        self.port_rc = torch.tensor(np.stack([rows, cols]).astype(np.int32), device=device)
        self.io = torch.tensor(topology.io_state_mask.astype(np.uint8), device=device)
        self.owm = torch.tensor(topology.out_weight_mask.astype(np.uint8), device=device)
        self.grid = (H, W)

    @classmethod
    def get(cls, topology, roi_bbox, device):
        key = (id(topology), topology, roi_bbox, str(device))
        g = cls._cache.get(key)
        if g is None:
            g = cls._cache[key] = cls(topology, roi_bbox, device)
        return g


class _CoddFuse(torch.autograd.Function):
    """Autograd node of the pre-step fusion: cell_params -> (w_eff, s_eff, b_roi,
    border_patch, port_params); s_prob, border_2d and w_pinned are non-differentiable
    side outputs."""

    @staticmethod
    def forward(ctx, cell, geo, mode, inv_tau, thr, hard_pin, act, slope):
        if not cell.is_cuda or cell.dtype != torch.float32:
            raise NeurocellError("cell_params must be a float32 device tensor")
        cell = cell.contiguous()
        dev = cell.device
        f = dict(device=dev, dtype=torch.float32)
        H, W = geo.grid
        w_eff = torch.empty(geo.h, geo.w, **f)
        s_eff = torch.empty(geo.h, geo.w, **f)
        b_roi = torch.empty(geo.h, geo.w, **f)
        patch = torch.empty(geo.Hp, geo.Wp, **f)
        pp = torch.empty(3, geo.P, **f)
        s_prob = torch.empty(H, W, **f)
        b2d = torch.empty(H, W, **f)
        wpin = torch.empty(H, W, **f)
        call("nc_codd_fuse_fwd", stream_ptr(), geo.chip, ptr(cell), ptr(geo.io), ptr(geo.owm),
             _abi.CODD_IDS[mode], inv_tau, thr, int(hard_pin), act, slope, geo.P,
             ptr(geo.port_rc), ptr(w_eff), ptr(s_eff), ptr(b_roi), ptr(patch), ptr(pp),
             ptr(s_prob), ptr(b2d), ptr(wpin))
        ctx.save_for_backward(cell)
        ctx.args = (geo, mode, inv_tau, thr, hard_pin, act, slope)
        ctx.mark_non_differentiable(s_prob, b2d, wpin)
        return w_eff, s_eff, b_roi, patch, pp, s_prob, b2d, wpin

    @staticmethod
    def backward(ctx, g_weff, g_seff, g_broi, g_patch, g_pp, *_):
        (cell,) = ctx.saved_tensors
        geo, mode, inv_tau, thr, hard_pin, act, slope = ctx.args
        g_cell = torch.empty_like(cell)
        c = lambda t: None if t is None else t.contiguous()
        call("nc_codd_fuse_bwd", stream_ptr(), geo.chip, ptr(cell), ptr(geo.io), ptr(geo.owm),
             _abi.CODD_IDS[mode], inv_tau, thr, int(hard_pin), act, slope, geo.P,
             ptr(geo.port_rc), None, None, ptr(c(g_weff)), ptr(c(g_seff)), ptr(c(g_broi)),
             ptr(c(g_patch)), ptr(c(g_pp)), None, None, ptr(g_cell))
        return g_cell, None, None, None, None, None, None, None


def precompute_step_params(params: VNNParams, topology: ChipTopology2D, activate="tanh",
                           sharpen_weights_fn=None, hard_pin_io: bool = False, roi_bbox=None,
                           codd_mode: str = "continuous", state_temperature: float = 1.0,
                           active_threshold: float = 0.6) -> PrecomputedStepParams:
    """params.py:220-322 on the gfx950 Codd-fusion kernel (differentiable w.r.t.
    ``params.cell_params``)."""
    _check_mode(codd_mode)
    if sharpen_weights_fn is not None:
        raise NeurocellError("sharpen_weights_fn is not part of the MI355X path")
    a, slope = act_id(activate)
    geo = _Geometry.get(topology, roi_bbox, params.cell_params.device)
    (w_eff, s_eff, b_roi, patch, pp, s_prob, b2d, wpin) = _CoddFuse.apply(
        params.cell_params, geo, codd_mode, inv_tau_f32(state_temperature),
        float(active_threshold), bool(hard_pin_io), a, slope)
    oh, ow = geo.out_size
    return PrecomputedStepParams(
        w_eff_roi=w_eff, s_eff_roi=s_eff, b_roi=b_roi, border_2d=b2d,
        w_eff_out=pp[0].reshape(oh, ow), s_eff_out=pp[1].reshape(oh, ow),
        b_out=pp[2].reshape(oh, ow), w_pinned=wpin, b_full=params.cell_params[1],
        s_prob=s_prob, border_patch=patch, port_params=pp)


def compute_codd_state_probs(s_raw: torch.Tensor, io_state_mask, hard_pin_io: bool = False,
                             codd_mode: str = "continuous", state_temperature: float = 1.0,
                             active_threshold: float = 0.6) -> torch.Tensor:
    """params.py:31-80: Codd probabilities on (H, W), differentiable w.r.t. ``s_raw``.

    Runs the fusion kernel on a degenerate chip (1x1 kernel, one direction, ROI = grid) whose
    s_eff equals s_prob, so value and straight-through gradient come from the same code as the
    propagation step."""
    _check_mode(codd_mode)
    H, W = s_raw.shape
    dev = s_raw.device
    key = ("codd_probs", H, W, str(dev), np.asarray(io_state_mask, dtype=bool).tobytes())
    geo = _Geometry._cache.get(key)
    if geo is None:
        from .topology import CoordinatePortSpec
        io = np.asarray(io_state_mask.cpu() if torch.is_tensor(io_state_mask) else io_state_mask,
                        dtype=bool)
        geo = _Geometry.__new__(_Geometry)
        geo.chip = _abi.ChipDesc(H, W, 1, 1, 1, 0, 0, H, W, 0, H, 0, W)
        geo.h, geo.w, geo.Hp, geo.Wp = H, W, H, W
        geo.P, geo.out_size, geo.grid = 0, (0, 1), (H, W)
        geo.port_rc = torch.zeros(2, 1, dtype=torch.int32, device=dev)
        geo.io = torch.tensor(io.astype(np.uint8), device=dev)
        geo.owm = torch.zeros(H, W, dtype=torch.uint8, device=dev)
        _Geometry._cache[key] = geo
    zeros = torch.zeros_like(s_raw)
    cell = torch.stack([zeros, zeros, s_raw])
    out = _CoddFuse.apply(cell, geo, codd_mode, inv_tau_f32(state_temperature),
                          float(active_threshold), bool(hard_pin_io), 0, 0.0)
    return out[1]  # s_eff = s_prob / M with M = 1

"""Adaptive active-region bucketing (piece 4): adaptive_mask.py of the reference.

``compute_adaptive_spatial_mask`` (:318-481) keeps its signature.  The per-epoch statistics
(effective filter radii, salience z-scores, seed mask, rectangular dilation, bounding box;
``_compute_adaptive_mask_tensors`` :200-315) run in one gfx950 workgroup
(``nc_adaptive_stats``); the 8 resulting integers are the only device->host crossing, and
the bucket quantisation (:105-161), hysteresis (:439-458) and cropped-topology view
(:164-197) are host integer logic restated here.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np
import torch

from . import _abi
from ._lib import call, ptr, stream_ptr
from .topology import ChipTopology2D, CoordinatePortSpec, PortSpec, _next_power_of_two

TILED_BLOCK_N = 1024


def _select_tile_block_n(n_pix: int, max_block_n: int = TILED_BLOCK_N) -> int:
    """kernels_pallas.py:65-73."""
    for cand in (1024, 512, 256, 128):
        if cand <= max_block_n and n_pix % cand == 0:
            return cand
    return max_block_n


@dataclass(frozen=True)
class AdaptiveMaskSpec:
    """adaptive_mask.py:37-55."""
    roi_bbox: tuple
    grid_bbox: tuple
    active_shape: tuple
    active_mask_roi: object
    cropped_mask_roi: object
    tile_mask: object
    eff_kernel_radii: tuple
    active_fraction: float
    salient_cell_count: int
    is_full_roi: bool
    cropped_topology: ChipTopology2D
    fft_shape: tuple
    raw_roi_bbox: tuple | None = None


def _quantize_interval(lo: int, hi: int, max_len: int, bucket_multiple: int) -> tuple:
    """adaptive_mask.py:105-161: expand [lo, hi) to a bucket multiple, centred and snapped to
    half-bucket (then quarter-bucket) aligned starts."""
    lo = max(0, min(lo, max_len - 1))
    hi = max(lo + 1, min(hi, max_len))
    raw_len = hi - lo
    if bucket_multiple <= 1 or raw_len >= max_len:
        return 0, max_len
    q_len = min(max_len, ((raw_len + bucket_multiple - 1) // bucket_multiple) * bucket_multiple)
    if q_len >= max_len or (max_len - q_len) < bucket_multiple:
        return 0, max_len
    ideal_lo = lo - 0.5 * (q_len - raw_len)
    min_valid_lo = max(0, hi - q_len)
    max_valid_lo = min(lo, max_len - q_len)

    def closest(step):
        first = ((min_valid_lo + step - 1) // step) * step
        if first > max_valid_lo:
            return None
        best, best_d = first, abs(first - ideal_lo)
        c = first + step
        while c <= max_valid_lo:
            d = abs(c - ideal_lo)
            if d < best_d:  # strict: the first (smallest) start wins ties
                best, best_d = c, d
            c += step
        return best

    new_lo = closest(max(1, bucket_multiple // 2))
    if new_lo is None:
        new_lo = closest(max(1, bucket_multiple // 4))
    if new_lo is None:
        new_lo = max(min_valid_lo, min(int(round(ideal_lo)), max_valid_lo))
    return int(new_lo), int(new_lo + q_len)


def _build_cropped_topology(topology: ChipTopology2D, r0, r1, c0, c1):
    """adaptive_mask.py:164-197."""
    h_act, w_act = r1 - r0, c1 - c0
    kh, kw = topology.kernel_size
    fft_shape = (_next_power_of_two(h_act + kh - 1), _next_power_of_two(w_act + kw - 1))
    if isinstance(topology.out_port, CoordinatePortSpec):
        ro_rows, ro_cols = topology.roi_out_offset
        off = (tuple(int(r - r0) for r in ro_rows), tuple(int(c - c0) for c in ro_cols))
    else:
        ro_r, ro_c = topology.roi_out_offset
        off = (int(ro_r - r0), int(ro_c - c0))
    return replace(topology, roi_shape=(h_act, w_act), roi_out_offset=off,
                   fft_shape=fft_shape), fft_shape


def _stats(params, topology: ChipTopology2D, margin_h, margin_w, salience_threshold,
           bias_threshold, filter_threshold, activity_map, activity_threshold):
    H, W = topology.grid_shape
    rh, rw = topology.pad_h, topology.pad_w
    roi_h, roi_w = topology.roi_shape
    kh, kw = topology.kernel_size
    dev = params.cell_params.device
    chip = _abi.ChipDesc(H, W, kh, kw, topology.directions, rh, rw, roi_h, roi_w, 0, roi_h, 0,
                         roi_w)
    io_roi = torch.tensor(topology.io_state_mask[rh:H - rh, rw:W - rw].astype(np.uint8),
                          device=dev)
    act = None
    if activity_map is not None:
        a = activity_map
        if tuple(a.shape) == (H, W):
            a = a[rh:H - rh, rw:W - rw]
        act = a.to(device=dev, dtype=torch.float32).contiguous()
    stats = torch.empty(8, device=dev, dtype=torch.int32)
    dil = torch.empty(roi_h, roi_w, device=dev, dtype=torch.uint8)
    call("nc_adaptive_stats", stream_ptr(), chip, ptr(params.cell_params.contiguous()),
         ptr(params.greens_filters.contiguous()), ptr(io_roi), ptr(act), int(margin_h),
         int(margin_w), float(salience_threshold), float(bias_threshold),
         float(filter_threshold), float(activity_threshold), ptr(stats), ptr(dil))
    return stats.cpu().numpy(), dil  # the per-epoch host sync (adaptive_mask.py:424)


def estimate_effective_filter_radii(greens_filters, threshold: float = 0.05) -> tuple:
    """adaptive_mask.py:58-81 (host restatement over the filter taps)."""
    g = greens_filters.detach().abs().amax(dim=0)[0].cpu().numpy()
    kh, kw = g.shape
    active = g >= threshold * g.max() + 1e-12
    rr = np.abs(np.arange(kh) - (kh - 1) // 2)[:, None]
    cc = np.abs(np.arange(kw) - (kw - 1) // 2)[None, :]
    return max(1, int(np.where(active, rr, 0).max())), max(1, int(np.where(active, cc, 0).max()))


def compute_adaptive_spatial_mask(params, topology: ChipTopology2D, margin=4,
                                  bucket_multiple: int = 8, salience_threshold: float = 2.5,
                                  bias_threshold: float = 0.05, filter_threshold: float = 0.05,
                                  activity_map=None, activity_threshold: float = 1e-3,
                                  prev_mask: AdaptiveMaskSpec | None = None) -> AdaptiveMaskSpec:
    """adaptive_mask.py:318-481."""
    margin_h, margin_w = (int(margin), int(margin)) if isinstance(margin, int) else (
        int(margin[0]), int(margin[1]))
    H, W = topology.grid_shape
    rh, rw = topology.pad_h, topology.pad_w
    roi_h, roi_w = topology.roi_shape
    n_pix = roi_h * roi_w
    block_n = _select_tile_block_n(n_pix, TILED_BLOCK_N)
    num_tiles = (n_pix + block_n - 1) // block_n
    dev = params.cell_params.device
    is_full_grid_out = (isinstance(topology.out_port, PortSpec)
                        and topology.out_port.size == topology.grid_shape)
    if is_full_grid_out and activity_map is None:
        radii = estimate_effective_filter_radii(params.greens_filters, filter_threshold)
        full = torch.ones(roi_h, roi_w, dtype=torch.bool, device=dev)
        return AdaptiveMaskSpec(
            roi_bbox=(0, roi_h, 0, roi_w), grid_bbox=(rh, H - rh, rw, W - rw),
            active_shape=(roi_h, roi_w), active_mask_roi=full, cropped_mask_roi=full,
            tile_mask=torch.ones(num_tiles, dtype=torch.bool, device=dev),
            eff_kernel_radii=radii, active_fraction=1.0, salient_cell_count=int(n_pix),
            is_full_roi=True, cropped_topology=topology, fft_shape=topology.fft_shape)
    st, dil = _stats(params, topology, margin_h, margin_w, salience_threshold, bias_threshold,
                     filter_threshold, activity_map, activity_threshold)
    r_eff_h, r_eff_w, salient, any_active = int(st[0]), int(st[1]), int(st[2]), bool(st[3])
    if any_active:
        r0_raw, r1_raw, c0_raw, c1_raw = (int(v) for v in st[4:8])
    else:
        r0_raw, r1_raw, c0_raw, c1_raw = 0, roi_h, 0, roi_w
    if prev_mask is not None:
        raw_prev = prev_mask.raw_roi_bbox if prev_mask.raw_roi_bbox is not None \
            else prev_mask.roi_bbox
        r0_raw, r1_raw = min(r0_raw, raw_prev[0]), max(r1_raw, raw_prev[1])
        c0_raw, c1_raw = min(c0_raw, raw_prev[2]), max(c1_raw, raw_prev[3])
    raw_bbox = (r0_raw, r1_raw, c0_raw, c1_raw)
    if prev_mask is not None and prev_mask.roi_bbox[0] <= r0_raw and r1_raw <= prev_mask.roi_bbox[1]:
        r0, r1 = prev_mask.roi_bbox[0], prev_mask.roi_bbox[1]
    else:
        r0, r1 = _quantize_interval(r0_raw, r1_raw, roi_h, bucket_multiple)
    if prev_mask is not None and prev_mask.roi_bbox[2] <= c0_raw and c1_raw <= prev_mask.roi_bbox[3]:
        c0, c1 = prev_mask.roi_bbox[2], prev_mask.roi_bbox[3]
    else:
        c0, c1 = _quantize_interval(c0_raw, c1_raw, roi_w, bucket_multiple)
    h_act, w_act = r1 - r0, c1 - c0
    cropped, fft_shape = _build_cropped_topology(topology, r0, r1, c0, c1)
    flat = dil.reshape(-1).bool()
    pad = num_tiles * block_n - n_pix
    if pad:
        flat = torch.cat([flat, torch.zeros(pad, dtype=torch.bool, device=dev)])
    tile_mask = flat.reshape(num_tiles, block_n).any(dim=1)
    return AdaptiveMaskSpec(
        roi_bbox=(r0, r1, c0, c1), grid_bbox=(rh + r0, rh + r1, rw + c0, rw + c1),
        active_shape=(h_act, w_act), active_mask_roi=dil.bool(),
        cropped_mask_roi=dil.bool()[r0:r1, c0:c1], tile_mask=tile_mask,
        eff_kernel_radii=(r_eff_h, r_eff_w), active_fraction=float(h_act * w_act) / float(n_pix),
        salient_cell_count=salient, is_full_roi=(h_act == roi_h and w_act == roi_w),
        cropped_topology=cropped, fft_shape=fft_shape, raw_roi_bbox=raw_bbox)

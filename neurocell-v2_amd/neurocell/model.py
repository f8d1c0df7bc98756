"""Stateless ``VonNeumannNetwork`` (model.py:29-227) over the gfx950 propagation path.

Same constructor, ``init``/``apply``/``__call__``/``compute_spatial_mask``/
``effective_states``/``threshold_states`` and the legacy ``.npz`` checkpoint format (keys
``weights``, ``biases``, ``states``, ``filters`` (1,Kh,Kw,M) IHWO, ``N``, ``depth``,
``kernel_size``, ``directions`` and any extra metadata).
"""
from __future__ import annotations

from typing import Sequence

import numpy as np
import torch

from .adaptive_mask import AdaptiveMaskSpec, compute_adaptive_spatial_mask
from .params import VNNParams, compute_codd_state_probs, init_vnn_params
from .propagator import propagate_vnn_2d
from .topology import ChipTopology2D


def sharpen_kernel(norm: bool = True) -> np.ndarray:
    """filters.py:56-68: the 3x3 sharpening stencil (centre 5, edge neighbours -1), divided
    by 5 when ``norm``."""
    k = np.array([[0, -1, 0], [-1, 5, -1], [0, -1, 0]], np.float32)
    return k / np.float32(5.0) if norm else k


class VonNeumannNetwork:
    """model.py:29-159.  ``apply(params, inputs)`` returns the output-port predictions
    (B, out_h, out_w); only the port cells of the last step are evaluated."""

    def __init__(self, topology: ChipTopology2D, activate="tanh", final_activate=None,
                 norm: bool = True, sharpen: bool = False, gated_filters: bool = False,
                 hard_pin_io: bool = False, backend: str = "nchw_direct", dtype=torch.float32,
                 codd_mode: str = "continuous", state_temperature: float = 1.0,
                 active_threshold: float = 0.6):
        self.topology = topology
        self.activate = activate
        self.final_activate = final_activate
        self.norm = norm
        self.sharpen = sharpen
        self.gated_filters = gated_filters
        self.hard_pin_io = hard_pin_io
        self.backend = backend
        self.dtype = dtype
        self.codd_mode = codd_mode
        self.state_temperature = state_temperature
        self.active_threshold = active_threshold
        # the weight-sharpening pre-filter (model.py:65-67): filters.sharpen, normalised
        self.sharpen_filter = sharpen_kernel(norm=True) if sharpen else None

    def init(self, rng, clear_outside_io: bool = False, legacy_compat: bool = True,
             device=None) -> VNNParams:
        """model.py:70-84: packed VNNParams on the device (``rng``: int seed or
        torch.Generator)."""
        return init_vnn_params(rng, self.topology, dtype=self.dtype,
                               clear_outside_io=clear_outside_io, legacy_compat=legacy_compat,
                               device=device)

    def compute_spatial_mask(self, params: VNNParams, margin=4, bucket_multiple: int = 8,
                             prev_mask: AdaptiveMaskSpec | None = None,
                             **kwargs) -> AdaptiveMaskSpec:
        """model.py:86-105: the pre-epoch active-region bucket for the next epoch."""
        return compute_adaptive_spatial_mask(params=params, topology=self.topology,
                                             margin=margin, bucket_multiple=bucket_multiple,
                                             prev_mask=prev_mask, **kwargs)

    def _resolve(self, codd_mode, state_temperature, active_threshold):
        return (self.codd_mode if codd_mode is None else codd_mode,
                self.state_temperature if state_temperature is None else state_temperature,
                self.active_threshold if active_threshold is None else active_threshold)

    def apply(self, params: VNNParams, inputs: torch.Tensor | Sequence[torch.Tensor],
              return_universe: bool = False, spatial_mask: AdaptiveMaskSpec | None = None,
              codd_mode: str | None = None, state_temperature: float | None = None,
              active_threshold: float | None = None):
        """model.py:107-139."""
        mode, tau, thr = self._resolve(codd_mode, state_temperature, active_threshold)
        return propagate_vnn_2d(params=params, inputs=inputs, topology=self.topology,
                                activate=self.activate, final_activate=self.final_activate,
                                norm=self.norm, sharpen_filter=self.sharpen_filter,
                                gated_filters=self.gated_filters, hard_pin_io=self.hard_pin_io,
                                backend=self.backend, return_universe=return_universe,
                                spatial_mask=spatial_mask, codd_mode=mode,
                                state_temperature=tau, active_threshold=thr)

    def __call__(self, params, inputs, return_universe: bool = False, spatial_mask=None,
                 codd_mode=None, state_temperature=None, active_threshold=None):
        """Alias for ``apply`` (model.py:141-162)."""
        return self.apply(params, inputs, return_universe=return_universe,
                          spatial_mask=spatial_mask, codd_mode=codd_mode,
                          state_temperature=state_temperature,
                          active_threshold=active_threshold)

    def effective_states(self, params: VNNParams, codd_mode: str | None = None,
                         state_temperature: float | None = None,
                         active_threshold: float | None = None) -> torch.Tensor:
        """model.py:164-185: Codd probabilities on (H, W) after IO pinning and gating."""
        mode, tau, thr = self._resolve(codd_mode, state_temperature, active_threshold)
        return compute_codd_state_probs(params.states, self.topology.io_state_mask,
                                        hard_pin_io=self.hard_pin_io, codd_mode=mode,
                                        state_temperature=tau, active_threshold=thr)

    @staticmethod
    def threshold_states(states_raw: torch.Tensor, active_threshold: float = 0.6):
        """model.py:187-197: 2 where s >= threshold, 1 where 0 < s < threshold, else s."""
        s = torch.where(states_raw >= active_threshold, torch.full_like(states_raw, 2.0),
                        states_raw)
        return torch.where((s > 0.0) & (s < active_threshold), torch.ones_like(s), s)

    def save_checkpoint(self, filename: str, params: VNNParams, **extra_metadata):
        """model.py:199-218: legacy-key ``.npz`` (filters in (1,Kh,Kw,M) IHWO)."""
        host = lambda t: t.detach().to("cpu").numpy()
        np.savez(filename, weights=host(params.weights), biases=host(params.biases),
                 states=host(params.states), filters=host(params.filters_ihwo.contiguous()),
                 N=self.topology.N, depth=self.topology.depth,
                 kernel_size=np.asarray(self.topology.kernel_size),
                 directions=self.topology.directions, **extra_metadata)

    @staticmethod
    def load_checkpoint(filename: str, device=None) -> VNNParams:
        """model.py:220-227: packed VNNParams from a legacy ``.npz`` (no pickles are read).
        Tensors land on ``device`` (default: the current HIP device when one is visible)."""
        with np.load(filename, allow_pickle=False) as data:
            w = torch.from_numpy(np.asarray(data["weights"], np.float32))
            b = torch.from_numpy(np.asarray(data["biases"], np.float32))
            s = torch.from_numpy(np.asarray(data["states"], np.float32))
            f_ihwo = torch.from_numpy(np.asarray(data["filters"], np.float32))
        if device is None:
            device = torch.device("cuda") if torch.cuda.is_available() else torch.device("cpu")
        cell = torch.stack([w, b, s]).to(device)
        filt = f_ihwo.permute(3, 0, 1, 2).contiguous().to(device)
        return VNNParams(cell_params=cell, greens_filters=filt)

"""Step executor: the VNN propagation step (propagator.py:209-682) and its reverse pass as a
fixed sequence of C-ABI launches over persistent device buffers.

A ``StepPlan`` is built once per (topology, batch size, active sub-ROI, activations) bucket --
the analogue of the reference's per-bbox jit cache (trainer.py:164-248).  It owns every
intermediate in HBM (laid out NCHW, fp32; spectra complex64 as (fft_h, fft_w/2+1)), so a
forward, a backward or a whole train step allocates nothing and issues no memset: callers may
capture it in a HIP graph (``torch.cuda.CUDAGraph``) and replay it.

Forward (pure ROI + hoisted border theorem, propagator.py:1-9, 343-682):
    codd fusion -> filter spectrum -> border-patch spectrum -> inject ->
    d-1 x [spectral conv -> hidden epilogue] -> spectral conv -> port epilogue
The hoisted border conv's delta, added to every step t >= 1's conv output, is folded into
those steps' correlations: the border patch's spectrum, phase-shifted from the VALID window
onto the ROI window, is added to their cell spectra (z + delta = irfft2((xhat + phat) ghat)),
so the epilogues see z + delta with no border term and the steps' dG carries the border's.
Reverse: port bwd -> d x [spectral conv bwd (dx, dG in the frequency domain)
    -> hidden epilogue bwd] -> filter-spectrum bwd -> border conv bwd -> codd fusion bwd.
The border conv's cotangent sum_{t>=1} sum_b gz_t is formed in the frequency domain by the
steps' dG reductions (linearity of rfft2), so the cotangent planes are not re-read for it.

Small filters (kh * kw <= 64, e.g. the 3 x 3 Game-of-Life and CLP chips) take the direct
correlation instead (propagator.py:373-386), whose spectral grid would be mostly padding:
    codd fusion -> inject -> border conv (VALID, B = 1) ->
    d-1 x [direct conv -> hidden epilogue (+ delta)] -> direct conv -> port epilogue (+ delta)
Reverse: port bwd (-> border cotangent) -> d x [direct conv bwd (dx, dG partial rows)
    -> hidden epilogue bwd (+= border cotangent)] -> border conv bwd -> dG row sum ->
    codd fusion bwd.
"""
from __future__ import annotations

import copy

import numpy as np
import torch

from . import _abi
from ._lib import NeurocellError, call, lib, ptr, stream_ptr, require_device
from .topology import ChipTopology2D, CoordinatePortSpec

_WAVE_FFT = (16, 32, 64)        # wavefront transforms (a plane per lane group)
# filters up to this many taps run the direct correlation (the reference's rule,
# propagator.py:373-386); a train step only with at least 4 directions and up to 36 taps (or
# up to 64 where the spectral grid is not a fused one), where its spatial reverse (input and
# filter gradients) measured faster than the spectral one on MI355X (bench.py --conv-compare)
_DIRECT_MAX_K = 64
_DIRECT_MAX_K_TRAIN = 36
_DIRECT_MIN_M_TRAIN = 4
_LARGE_FFT = (64, 128, 256)     # workgroup transforms over LDS segments


def spectral_grid_supported(fh: int, fw: int) -> bool:
    """True when the C ABI has kernels for an (fh, fw) spectral grid."""
    return ((fh in _WAVE_FFT and fw in _WAVE_FFT)
            or (fh in _LARGE_FFT and fw in _LARGE_FFT))


def _npow2(x: int) -> int:
    return 1 << (int(x) - 1).bit_length()


def act_id(activate) -> tuple[int, float]:
    """Maps an activation (name, None, or a callable with a matching ``__name__``) to the
    kernel id and leaky slope, as kernels_pallas.py:76-99 resolves it."""
    if activate is None:
        return _abi.ACT_IDS["identity"], 1.0
    if isinstance(activate, str):
        name = activate
    else:
        name = getattr(activate, "__name__", "")
        kw = getattr(activate, "keywords", None)
        if name == "" and getattr(activate, "func", None) is not None:
            name = getattr(activate.func, "__name__", "")
        if name == "leaky_relu" and kw:
            return _abi.ACT_IDS["leaky_relu"], float(kw.get("negative_slope", 0.01))
    if name not in _abi.ACT_IDS:
        raise ValueError(f"Unsupported activation function: {activate}")
    return _abi.ACT_IDS[name], (0.01 if name == "leaky_relu" else 0.0)


def port_input_shapes(inputs, topology: ChipTopology2D) -> list:
    """Per-port (ih, iw) as written into the grid (propagator.py:88-100, 124-130: a 3-D
    per-port input is written with its own shape)."""
    if isinstance(inputs, (list, tuple)):
        arrs = list(inputs)
        shapes = []
        for a, p in zip(arrs, topology.in_ports):
            if isinstance(p, CoordinatePortSpec):
                shapes.append((p.num_points, 1))
            elif a.ndim == 3:
                shapes.append((int(a.shape[1]), int(a.shape[2])))
            else:
                shapes.append(tuple(p.size))
        return shapes
    if len(topology.in_ports) == 1:
        p = topology.in_ports[0]
        if inputs.ndim == 2 or (inputs.ndim == 3 and tuple(inputs.shape[1:]) == tuple(p.size)):
            if isinstance(p, CoordinatePortSpec):
                return [(p.num_points, 1)]
            return [tuple(inputs.shape[1:]) if inputs.ndim == 3 else tuple(p.size)]
    shapes = []
    for i, p in enumerate(topology.in_ports):
        if isinstance(p, CoordinatePortSpec):
            shapes.append((p.num_points, 1))
        else:
            sub = inputs[:, i]
            shapes.append((int(sub.shape[1]), int(sub.shape[2])) if sub.ndim == 3
                          else tuple(p.size))
    return shapes


def flatten_inputs(inputs, topology: ChipTopology2D) -> torch.Tensor:
    """Concatenates the per-port inputs into one (B, n_in) fp32 device tensor."""
    if isinstance(inputs, (list, tuple)):
        parts = [a.reshape(a.shape[0], -1) for a in inputs]
    elif len(topology.in_ports) == 1 and (inputs.ndim == 2 or (
            inputs.ndim == 3 and tuple(inputs.shape[1:]) == tuple(topology.in_ports[0].size))):
        parts = [inputs.reshape(inputs.shape[0], -1)]
    else:
        parts = [inputs[:, i].reshape(inputs.shape[0], -1)
                 for i in range(len(topology.in_ports))]
    x = torch.cat(parts, dim=1) if len(parts) > 1 else parts[0]
    if x.dtype != torch.float32:
        raise NeurocellError(f"inputs must be float32, got {x.dtype}")
    if not x.is_cuda:
        raise NeurocellError("inputs must already be resident on the device")
    return x.contiguous()


class StepPlan:
    """Launch plan and persistent buffers for one (topology, B, sub-ROI) bucket."""

    def __init__(self, topology: ChipTopology2D, batch_size: int, port_shapes: list,
                 roi_bbox=None, activate="tanh", final_activate=None, hard_pin_io=False,
                 training=True, device=None, gated_filters=False, sharpen=None,
                 universe=False, conv="auto"):
        self.device = device or require_device()
        self.topo = topology
        self.B = int(batch_size)
        self.training = bool(training)
        self.hard_pin_io = bool(hard_pin_io)
        # gated filters (propagator.py:266-267): the steps use sigmoid(filters)
        self.gated = bool(gated_filters)
        # weight sharpening (params.py:246-247): the Codd fusion sees corr_SAME(W, kernel)
        self.sharpen = None if sharpen is None else np.ascontiguousarray(sharpen, np.float32)
        # the full-grid output path (propagator.py:684-734): return_universe, or an output
        # port outside the ROI (allow_border_output, full-grid ports), reads the port from the
        # final universe
        self.universe = bool(universe) or not topology.out_in_roi
        self.want_universe = bool(universe)
        self.act, self.slope = act_id(activate)
        self.fact, self.fslope = act_id(final_activate)
        H, W = topology.grid_shape
        kh, kw = topology.kernel_size
        M, d = topology.directions, topology.depth
        roi_h, roi_w = topology.roi_shape
        r0, r1, c0, c1 = roi_bbox if roi_bbox is not None else (0, roi_h, 0, roi_w)
        self.bbox = (int(r0), int(r1), int(c0), int(c1))
        self.cropped = roi_bbox is not None and self.bbox != (0, roi_h, 0, roi_w)
        h, w = r1 - r0, c1 - c0
        self.H, self.W, self.kh, self.kw, self.M, self.d = H, W, kh, kw, M, d
        self.h, self.w, self.N = h, w, h * w
        # padding modes (propagator.py:276-341): VALID adds the hoisted border conv to steps
        # t >= 1; SAME and CIRCULAR take the whole grid as the ROI with no border term, SAME
        # zero-padding the correlation and CIRCULAR wrapping it round the grid
        self.mode = topology.padding_mode
        self.circular = self.mode == "CIRCULAR"
        self.border = self.mode == "VALID" and d > 1
        # the correlation: spectral, or direct for small filters (propagator.py:373-386 uses a
        # direct conv for kh * kw <= 64), whose FFT grid would be mostly padding
        if conv not in ("auto", "spectral", "direct"):
            raise NeurocellError(f"conv must be 'auto', 'spectral' or 'direct', got {conv!r}")
        def fits(hin, win):  # the ROI steps, the full-grid t=0 step, the border conv
            return lib().nc_direct_conv_fits(M, hin, win, h, w, kh, kw, int(self.circular),
                                             int(self.training)) == 1
        direct_ok = (kh * kw <= _DIRECT_MAX_K and not (self.circular and self.cropped)
                     and fits(h, w) and fits(H, W)
                     and (not self.border or fits(h + kh - 1, w + kw - 1)))
        if conv == "direct" and not direct_ok:
            raise NeurocellError("the direct correlation takes kh * kw <= 64, M <= 64 and "
                                 "planes up to 256 wide whose bands fit the workgroup's LDS")
        auto = True
        if self.training:  # measured: the direct reverse pays up to 36 taps, or up to 64
            # where the spectral grid is not one of the fused 32x64 / 64x64 ones
            sg = (H, W) if self.circular else (
                (_npow2(h + kh - 1), _npow2(w + kw - 1)) if self.cropped
                else tuple(topology.fft_shape))
            sg = tuple(max(16, v) for v in sg)
            fused_grid = sg[1] == 64 and sg[0] in (32, 64)
            auto = M >= _DIRECT_MIN_M_TRAIN and (kh * kw <= _DIRECT_MAX_K_TRAIN or not fused_grid)
        self.direct = conv == "direct" or (conv == "auto" and direct_ok and auto)
        if self.direct:
            if self.circular and self.cropped:
                raise NeurocellError("adaptive crops are not supported in CIRCULAR mode")
            self.fft = None
        elif self.circular:
            if self.cropped:
                raise NeurocellError("adaptive crops are not supported in CIRCULAR mode")
            # the correlation is circular on the grid itself (topology.py:256-258)
            self.fft = (H, W)
            if not spectral_grid_supported(H, W):
                raise NeurocellError(f"CIRCULAR mode runs on the {H}x{W} grid itself: both "
                                     f"sides in {_WAVE_FFT} or both in {_LARGE_FFT}")
            if kh > H or kw > W:
                raise NeurocellError("the filter is larger than the circular grid")
        else:
            if self.cropped:
                self.fft = (_npow2(h + kh - 1), _npow2(w + kw - 1))  # adaptive_mask.py:177-180
            else:
                self.fft = tuple(topology.fft_shape)
            # a linear correlation is the same on any grid it fits: grids below 16 points
            # per axis run on 16
            self.fft = tuple(max(16, v) for v in self.fft)
            if not spectral_grid_supported(*self.fft):
                raise NeurocellError(f"spectral grid {self.fft} is not supported (both axes "
                                     f"in {_WAVE_FFT} or both in {_LARGE_FFT})")
            if h + kh - 1 > self.fft[0] or w + kw - 1 > self.fft[1]:
                raise NeurocellError("linear correlation does not fit the spectral grid")
        fh, fw = self.fft if self.fft else (0, 0)
        self.F = fh * (fw // 2 + 1)
        self.cp = ((kh - 1) // 2, (kw - 1) // 2)
        self.Hp, self.Wp = h + kh - 1, w + kw - 1
        # circular shift taking the border conv's VALID window (kh-1, kw-1) onto the ROI
        # steps' window cp: the patch spectrum shifted by it joins every ROI step's spectrum
        self.bshift = (((self.cp[0] - (kh - 1)) % fh, (self.cp[1] - (kw - 1)) % fw)
                       if self.fft else (0, 0))
        self.chip = _abi.ChipDesc(H, W, kh, kw, M, topology.pad_h, topology.pad_w, roi_h, roi_w,
                                  r0, r1, c0, c1)
        # output port cells
        rows, cols = topology.out_cells_roi()
        self.P = int(rows.size)
        self.out_size = tuple(topology.out_port.size)
        dev = self.device
        if self.universe:
            gr, gc = topology.out_cells_grid()
            if ((gr < 0) | (gr >= H) | (gc < 0) | (gc >= W)).any():
                raise NeurocellError("output port lies outside the grid")
            cells = (gr * W + gc).astype(np.int32)
            # port cells by grid cell for the reverse: first port at each cell, next port at
            # the same cell, in port order
            head = np.full(H * W, -1, np.int32)
            nxt = np.full(self.P, -1, np.int32)
            for k in range(self.P - 1, -1, -1):
                nxt[k] = head[cells[k]]
                head[cells[k]] = k
            self.port_cells = torch.tensor(cells, device=dev)
            self.port_head = torch.tensor(head, device=dev)
            self.port_next = torch.tensor(nxt, device=dev)
            rows = cols = np.zeros(0, np.int32)  # no port parameters on this path
        elif ((rows < r0) | (rows >= r1) | (cols < c0) | (cols >= c1)).any():
            raise NeurocellError("output port lies outside the active sub-ROI")
        self.n_pp = int(rows.size)  # cells with port parameters (the port path's)
        self.port_rc = torch.tensor(np.stack([rows, cols]).astype(np.int32), device=dev)
        # the port indices by ROI cell, for the reverse's gather of port-parameter gradients
        cell_of = (rows * roi_w + cols).astype(np.int64)
        order = np.argsort(cell_of, kind="stable")
        start = np.searchsorted(cell_of[order], np.arange(roi_h * roi_w + 1))
        self.pp_start = torch.tensor(start.astype(np.int32), device=dev)
        self.pp_list = torch.tensor(order.astype(np.int32), device=dev)
        flat = ((rows - r0) * w + (cols - c0)).astype(np.int32)
        self.port_idx = torch.tensor(flat, device=dev)
        # a port that is the whole (sub-)ROI in row-major order (the Game-of-Life universe
        # port): its epilogue is the hidden one with the port parameters and the final
        # activation, so it runs on the epilogue kernels at any size
        self.dense_port = (not self.universe and self.P == self.N
                           and np.array_equal(flat, np.arange(self.N)))
        if not self.dense_port and not self.universe and (self.P > 256 or M * self.P > 8192):
            raise NeurocellError(f"an output port of {self.P} cells must cover the whole ROI "
                                 "in row-major order (the port kernels gather at most 256 "
                                 "cells, 8192 per sample over the directions)")
        self.io_mask = torch.tensor(topology.io_state_mask.astype(np.uint8), device=dev)
        if self.sharpen is not None:
            sh, sw = self.sharpen.shape
            if sh % 2 == 0 or sw % 2 == 0 or sh > H or sw > W:
                raise NeurocellError(f"sharpen kernel {self.sharpen.shape} must be odd and fit "
                                     "the grid")
            self.sh_fft = tuple(max(16, _npow2(v)) for v in (H + sh - 1, W + sw - 1))
            if not spectral_grid_supported(*self.sh_fft):
                raise NeurocellError(f"the sharpening grid {self.sh_fft} is not supported")
        self.owm = torch.tensor(topology.out_weight_mask.astype(np.uint8), device=dev)
        # input injection map (gather form)
        self.port_shapes = [tuple(int(v) for v in s) for s in port_shapes]
        src, self.t0_grid = self._inject_map()
        self.n_in = int(sum(a * b for a, b in self.port_shapes))
        self.src = torch.tensor(src, device=dev)
        self._alloc()

    # ------------------------------------------------------------------ geometry helpers
    def _inject_map(self):
        """propagator.py:135-191: ROI gather map when every port fits the (cropped) ROI, else
        the full-grid t=0 map (propagator.py:347-352)."""
        t = self.topo
        r0, r1, c0, c1 = self.bbox
        min_r, max_r = t.pad_h + r0, t.pad_h + r1
        min_c, max_c = t.pad_w + c0, t.pad_w + c1
        fits = t.in_in_roi
        if fits:
            for port, (ih, iw) in zip(t.in_ports, self.port_shapes):
                if isinstance(port, CoordinatePortSpec):
                    if not all(min_r <= r < max_r and min_c <= c < max_c for r, c in port.coords):
                        fits = False
                else:
                    pr, pc = port.offset
                    if pr < min_r or pc < min_c or pr + ih > max_r or pc + iw > max_c:
                        fits = False
        if fits:
            base_r, base_c, hh, ww = min_r, min_c, self.h, self.w
        else:
            if self.cropped:
                raise NeurocellError("inputs outside a cropped sub-ROI are not supported")
            if self.fft and (self.H > self.fft[0] or self.W > self.fft[1]):
                raise NeurocellError("full-grid t=0 step does not fit the spectral grid")
            base_r, base_c, hh, ww = 0, 0, self.H, self.W
        src = np.full(hh * ww, -1, np.int32)
        e = 0
        for port, (ih, iw) in zip(t.in_ports, self.port_shapes):
            if isinstance(port, CoordinatePortSpec):
                for k, (r, c) in enumerate(port.coords):
                    src[(r - base_r) * ww + (c - base_c)] = e + k
                e += port.num_points
                continue
            pr, pc = port.offset
            for i in range(ih):
                for j in range(iw):
                    src[(pr - base_r + i) * ww + (pc - base_c + j)] = e + i * iw + j
            e += ih * iw
        return src, not fits

    def _alloc(self):
        if self.direct:
            return self._alloc_direct()
        dev, B, M, d, h, w, F = self.device, self.B, self.M, self.d, self.h, self.w, self.F
        f = dict(device=dev, dtype=torch.float32)
        c = dict(device=dev, dtype=torch.complex64)
        self.w_eff = torch.empty(h, w, **f)
        self.s_eff = torch.empty(h, w, **f)
        self.b_roi = torch.empty(h, w, **f)
        self.patch = torch.empty(self.Hp, self.Wp, **f)
        self.pp = torch.empty(3, self.n_pp, **f)
        self.ghat = torch.empty(M, F, **c)
        self.filt_g = torch.empty(M, 1, self.kh, self.kw, **f) if self.gated else None
        self._alloc_sharpen()
        self.border_hat = torch.empty(1, F, **c)  # shifted border-patch spectrum
        t0_shape = (B, self.H, self.W) if self.t0_grid else (B, h, w)
        self.x0 = torch.empty(*t0_shape, **f)
        nz = d if self.training else 1
        # step states t >= 1 as the epilogue's uncombined direction-group partials (G planes
        # per sample, summed by the next step's transform as it loads them)
        self.G = _abi_int("nc_fftconv_epilogue_partials", B, M, h, w, *self.fft)
        self.xs = [self.x0] + [torch.empty(self.G, B, h, w, **f) for _ in range(d - 1)]
        self.zs = [torch.empty(B, M, h, w, **f) for _ in range(nz)]
        # cell spectra: one per step for the reverse pass, one shared buffer for evaluation
        self.xhat = [torch.empty(B, F, **c) for _ in range(d if self.training else 1)]
        self.mean = [torch.empty(B, M, **f) for _ in range(d)]
        self.rstd = [torch.empty(B, M, **f) for _ in range(d)]
        self.out = torch.empty(B, self.P, **f)
        port_path = not (self.dense_port or self.universe)
        self.zo = torch.empty(B, M, self.P, **f) if port_path else None
        if not port_path:  # the last epilogue's direction-group partial outputs
            self.port_parts = torch.empty(self.G, B, h, w, **f)
        self.pre = torch.empty(B, self.P, **f) if self.fact != 0 and not self.universe else None
        if self.universe:
            self.s_prob = torch.empty(self.H, self.W, **f)
            self.univ = torch.empty(B, self.H, self.W, **f) if self.want_universe else None
        # on the 128/256-point grids the workspace also holds the two-pass correlation's
        # intermediate (the epilogue's scratch reuses it once z is written)
        n_ep = max(_abi_size("nc_epilogue_workspace_size", B, M, h, w),
                   _abi_size("nc_fftconv_port_workspace_size", B, M, h, w, *self.fft, self.P)
                   if port_path else 0,
                   lib().nc_fftconv_correlate_workspace_size(B, M, h, w, *self.fft))
        self.ws_epi = torch.empty(max(1, n_ep // 4), **f)
        if self.training:
            n_fc = max(_abi_size("nc_fftconv_bwd_workspace_size", B, M, *self.fft),
                       _abi_size("nc_fftconv_bwd_workspace_size", 1, M, *self.fft))
            self.ws_fc = torch.empty(max(1, n_fc // 4), **f)
            self.gz = torch.empty(B, M, h, w, **f)
            self.gy = [torch.empty(B, h, w, **f) for _ in range(2)]
            # frequency-domain gradient sums: the filter gradients (ROI steps, VALID full-grid
            # step) and the spectra of the border cotangent sum_b gz over the steps with the
            # border term, accumulated step by step as row stacks of the dG reductions' sample
            # chunks and summed once after the last step
            self.npart = _abi_int("nc_fftconv_bwd_partials", B, M, *self.fft)
            self.gdelta_hat = torch.empty(M, F, **c)
            self.dghat = torch.empty(M, F, **c)
            self.dghat_v = torch.empty(M, F, **c)
            if self.npart > 1:
                self.rows = {k: torch.empty(self.npart, M, F, **c) for k in ("dg", "dgv", "gd")}
            else:  # a single row is the sum itself
                self.rows = {"dg": self.dghat, "dgv": self.dghat_v, "gd": self.gdelta_hat}
            # parameter-gradient partial rows, summed in the same launch: R rows per hidden
            # epilogue step for each of gw / gs / gb, B rows per port parameter
            self.R = _abi_int("nc_epilogue_bwd_partials", B, M, h, w)
            # (the universe path's last epilogue takes a block of its own)
            self.n_epi = d - 1 + int(self.universe)
            self.pg_rows = torch.empty(3, max(1, self.n_epi) * self.R, h * w, **f)
            # port-parameter partial rows: B per parameter, or the epilogue's R for a dense port
            self.pp_rows = torch.empty(3, self.R if self.dense_port else B, self.n_pp, **f)
            if self.universe:
                self.g_roi = torch.empty(B, h, w, **f)
                self.g_sprob = torch.empty(self.H, self.W, **f)
                self.g_bfull = torch.empty(self.H, self.W, **f)
            self.g_pre = torch.empty(B, self.P, **f) if self.dense_port else None
            self.gw = torch.empty(h, w, **f)
            self.gs = torch.empty(h, w, **f)
            self.gb = torch.empty(h, w, **f)
            self.gpp = torch.empty(3, self.n_pp, **f)
            self.gpatch = torch.empty(self.Hp, self.Wp, **f)
            self.g_out = torch.empty(B, self.P, **f)
            self.loss = torch.empty(1, **f)

    def _alloc_sharpen(self):
        """The sharpening's filter spectrum and its buffers (both correlation paths run the
        SAME sharpening on its own spectral grid)."""
        if self.sharpen is None:
            return
        dev, H, W = self.device, self.H, self.W
        f = dict(device=dev, dtype=torch.float32)
        c = dict(device=dev, dtype=torch.complex64)
        fs = self.sh_fft[0] * (self.sh_fft[1] // 2 + 1)
        self.cell_s = torch.empty(3, H, W, **f)     # [sharpened W, B, S]
        self.sh_xhat = torch.empty(1, fs, **c)
        self.sh_ghat = torch.empty(1, fs, **c)
        self.sh_k = torch.from_numpy(self.sharpen).to(dev).reshape(1, 1, *self.sharpen.shape)
        call("nc_filter_spectrum_fwd", stream_ptr(), 1, *self.sharpen.shape, *self.sh_fft,
             ptr(self.sh_k), ptr(self.sh_ghat))
        if self.training:
            self.g_cell_s = torch.empty(3, H, W, **f)
            self.sh_dg = torch.empty(1, fs, **c)
            n_ws = _abi_size("nc_fftconv_bwd_workspace_size", 1, 1, *self.sh_fft)
            self.sh_ws = torch.empty(max(1, n_ws // 4), **f)

    def _alloc_common(self, G):
        """Buffers both correlation paths share: parameters, step states, z, statistics,
        port outputs and the reverse pass's gradient accumulators."""
        dev, B, M, d, h, w = self.device, self.B, self.M, self.d, self.h, self.w
        f = dict(device=dev, dtype=torch.float32)
        self.w_eff = torch.empty(h, w, **f)
        self.s_eff = torch.empty(h, w, **f)
        self.b_roi = torch.empty(h, w, **f)
        self.patch = torch.empty(self.Hp, self.Wp, **f)
        self.pp = torch.empty(3, self.n_pp, **f)
        self.filt_g = torch.empty(M, 1, self.kh, self.kw, **f) if self.gated else None
        self._alloc_sharpen()
        t0_shape = (B, self.H, self.W) if self.t0_grid else (B, h, w)
        self.x0 = torch.empty(*t0_shape, **f)
        self.G = G
        self.xs = [self.x0] + [torch.empty(G, B, h, w, **f) for _ in range(d - 1)]
        self.zs = [torch.empty(B, M, h, w, **f) for _ in range(d if self.training else 1)]
        self.mean = [torch.empty(B, M, **f) for _ in range(d)]
        self.rstd = [torch.empty(B, M, **f) for _ in range(d)]
        self.out = torch.empty(B, self.P, **f)
        port_path = not (self.dense_port or self.universe)
        self.zo = torch.empty(B, M, self.P, **f) if port_path else None
        if not port_path:
            self.port_parts = torch.empty(G, B, h, w, **f)
        self.pre = torch.empty(B, self.P, **f) if self.fact != 0 and not self.universe else None
        if self.universe:
            self.s_prob = torch.empty(self.H, self.W, **f)
            self.univ = torch.empty(B, self.H, self.W, **f) if self.want_universe else None
        self.n_epi = d - 1 + int(self.universe)
        if self.training:
            self.gz = torch.empty(B, M, h, w, **f)
            self.gy = [torch.empty(B, h, w, **f) for _ in range(2)]
            if self.universe:
                self.g_roi = torch.empty(B, h, w, **f)
                self.g_sprob = torch.empty(self.H, self.W, **f)
                self.g_bfull = torch.empty(self.H, self.W, **f)
            self.g_pre = torch.empty(B, self.P, **f) if self.dense_port else None
            self.gw = torch.empty(h, w, **f)
            self.gs = torch.empty(h, w, **f)
            self.gb = torch.empty(h, w, **f)
            self.gpp = torch.empty(3, self.n_pp, **f)
            self.gpatch = torch.empty(self.Hp, self.Wp, **f)
            self.g_out = torch.empty(B, self.P, **f)
            self.loss = torch.empty(1, **f)
        return port_path

    def _alloc_direct(self):
        """Buffers of the direct path: the hoisted border conv's delta (VALID), the filter
        gradient's partial rows (each step's bands, then the border conv's) and the border
        cotangent sum_b gz over the steps that carry the border term."""
        dev, B, M, d, h, w = self.device, self.B, self.M, self.d, self.h, self.w
        f = dict(device=dev, dtype=torch.float32)
        port_path = self._alloc_common(_abi_int("nc_epilogue_fwd_partials", B, M, h, w))
        self.delta = torch.empty(M, h, w, **f) if self.border else None
        self.ws_epi = torch.empty(max(1, _abi_size("nc_epilogue_workspace_size", B, M, h, w) // 4),
                                  **f)
        del port_path
        if self.training:
            K = self.kh * self.kw
            self.dg_step_rows = _abi_int("nc_direct_conv_dg_partials", B, M, h, w, self.kh,
                                         self.kw)
            self.dg_border_rows = (_abi_int("nc_direct_conv_dg_partials", 1, M, h, w, self.kh,
                                            self.kw) if self.border else 0)
            self.dg_rows = torch.empty(d * self.dg_step_rows + self.dg_border_rows, M * K, **f)
            self.gdelta = torch.empty(M, h, w, **f) if self.border else None

    def fresh(self) -> "StepPlan":
        """A plan sharing this one's static maps with its own activation buffers."""
        p = copy.copy(self)
        p._alloc()
        return p

    # ------------------------------------------------------------------ forward
    def forward(self, cell: torch.Tensor, filt: torch.Tensor, x_flat: torch.Tensor,
                codd_mode: str = "continuous", inv_tau: float = 1.0,
                active_threshold: float = 0.6) -> torch.Tensor:
        """Runs the d-step forward for inputs (B, n_in); returns the (B, P) port outputs."""
        s = stream_ptr()
        B, M, h, w = self.B, self.M, self.h, self.w
        fh, fw = self.fft if self.fft else (0, 0)
        if tuple(x_flat.shape) != (B, self.n_in):
            raise NeurocellError(f"inputs must be ({B}, {self.n_in}), got {tuple(x_flat.shape)}")
        mode = _abi.CODD_IDS[codd_mode]
        if self.sharpen is not None:  # the Codd fusion sees the sharpened weights
            ks = self.sharpen.shape
            self.cell_s[1:].copy_(cell[1:])
            call("nc_fftconv_fwd", s, 1, 1, self.H, self.W, self.H, self.W, (ks[0] - 1) // 2,
                 (ks[1] - 1) // 2, *self.sh_fft, ptr(cell[0]), ptr(self.sh_ghat),
                 ptr(self.cell_s[0]), ptr(self.sh_xhat))
            cell = self.cell_s
        # the Codd fusion and the input injection in one launch
        call("nc_step_prologue", s, self.chip, ptr(cell), ptr(self.io_mask), ptr(self.owm), mode,
             inv_tau, active_threshold, int(self.hard_pin_io), self.act, self.slope, self.n_pp,
             ptr(self.port_rc), ptr(self.w_eff), ptr(self.s_eff), ptr(self.b_roi),
             ptr(self.patch), ptr(self.pp), ptr(self.s_prob) if self.universe else None, B,
             self.n_in, ptr(x_flat), self.x0[0].numel(), ptr(self.src), ptr(self.x0))
        if self.gated:
            call("nc_filter_gate_fwd", s, self.filt_g.numel(), ptr(filt), ptr(self.filt_g))
            filt = self.filt_g
        if self.direct:
            return self._forward_direct(s, cell, filt)
        # the independent spectra in one call: filter spectra (kernels_greens.py:240-259), the
        # border patch's and the first step's cell spectra
        x0h, x0w = (self.H, self.W) if self.t0_grid else (h, w)
        xh0 = self.xhat[0]
        jobs = [(_addr(filt), _addr(self.ghat), None, M, self.kh, self.kw, 1, 0, 0),
                (_addr(self.x0), _addr(xh0), None, B, x0h, x0w, 0, 0, 0)]
        if self.border:
            # hoisted VALID border conv (propagator.py:362-366): its delta is added to every
            # step t >= 1's correlation, so the patch spectrum (shifted onto the ROI window)
            # joins those steps' cell spectra and their correlation yields z + delta directly
            jobs.append((_addr(self.patch), _addr(self.border_hat), None, 1, self.Hp, self.Wp, 0,
                         self.bshift[0], self.bshift[1]))
        call("nc_plane_spectra", s, fh, fw, len(jobs), _abi.spectrum_jobs(*jobs))
        # hidden steps: the correlation and the epilogue run as one kernel on the 32x64 and
        # 64x64 grids, where evaluation never materialises z
        fused = fw == 64 and fh in (32, 64)
        for t in range(self.d):
            last = t == self.d - 1
            z = self.zs[t if self.training else 0]
            xh = self.xhat[t if self.training else 0]
            if t == 0:
                if self.t0_grid:  # VALID full-grid step: its own spectral shift
                    r0, _, c0, _ = self.bbox
                    p0 = (self.kh - 1 + r0, self.kw - 1 + c0)
                else:
                    p0 = self.cp
                xh = xh0
            else:
                p0 = self.cp
                # z + delta comes out of the correlation: the border spectrum joins x's
                call("nc_fftconv_spectra", s, B, h, w, fh, fw, ptr(self.xs[t]), self.G,
                     ptr(self.border_hat) if self.border else None, ptr(xh))
            # z already holds z + delta: the epilogues run without their border term
            if not last:
                zk = None if fused and not self.training else z
                call("nc_fftconv_epilogue_fwd", s, B, M, h, w, p0[0], p0[1], fh, fw, ptr(xh),
                     ptr(self.ghat), self.act, self.slope, ptr(self.w_eff), ptr(self.s_eff),
                     ptr(self.b_roi), ptr(zk), ptr(self.xs[t + 1]), ptr(self.mean[t]),
                     ptr(self.rstd[t]), ptr(self.ws_epi), self.ws_epi.numel() * 4)
            elif self.universe:
                # the last epilogue with the final activation on the ROI parameters, then the
                # universe and the port read from it (propagator.py:684-734)
                zk = None if fused and not self.training else z
                call("nc_fftconv_epilogue_fwd", s, B, M, h, w, p0[0], p0[1], fh, fw, ptr(xh),
                     ptr(self.ghat), self.fact, self.fslope, ptr(self.w_eff), ptr(self.s_eff),
                     ptr(self.b_roi), ptr(zk), ptr(self.port_parts), ptr(self.mean[t]),
                     ptr(self.rstd[t]), ptr(self.ws_epi), self.ws_epi.numel() * 4)
                call("nc_universe_fwd", s, self.chip, B, self.G, int(self.mode == "VALID"),
                     self.fact, self.fslope, ptr(self.port_parts), _addr(cell) + 4 * self.H *
                     self.W, ptr(self.s_prob), self.P, ptr(self.port_cells), ptr(self.univ),
                     ptr(self.out))
            elif self.dense_port:
                zk = None if fused and not self.training else z
                call("nc_fftconv_epilogue_fwd", s, B, M, h, w, p0[0], p0[1], fh, fw, ptr(xh),
                     ptr(self.ghat), self.fact, self.fslope, ptr(self.pp[0]), ptr(self.pp[1]),
                     ptr(self.pp[2]), ptr(zk), ptr(self.port_parts), ptr(self.mean[t]),
                     ptr(self.rstd[t]), ptr(self.ws_epi), self.ws_epi.numel() * 4)
                call("nc_port_dense_fwd", s, B * self.P, self.G, self.fact, self.fslope,
                     ptr(self.port_parts), ptr(self.out), ptr(self.pre))
            else:
                # the correlation and the port statistics in one kernel on the 64-wide grids
                zk = None if fused and not self.training else z
                call("nc_fftconv_port_fwd", s, B, M, h, w, p0[0], p0[1], fh, fw, ptr(xh),
                     ptr(self.ghat), self.fact, self.fslope, self.P, ptr(self.port_idx),
                     ptr(self.pp), ptr(zk), ptr(self.out), ptr(self.zo), ptr(self.mean[t]),
                     ptr(self.rstd[t]), ptr(self.pre), ptr(self.ws_epi),
                     self.ws_epi.numel() * 4)
        return self.out

    def _conv_input(self, t):
        """(x, n_parts, hin, win, oh, ow) of step t's direct correlation."""
        kh, kw = self.kh, self.kw
        if t == 0:
            if self.t0_grid:  # VALID correlation of the full grid, read at the sub-ROI
                return self.x0, 1, self.H, self.W, self.bbox[0], self.bbox[2]
            return self.x0, 1, self.h, self.w, -((kh - 1) // 2), -((kw - 1) // 2)
        return self.xs[t], self.G, self.h, self.w, -((kh - 1) // 2), -((kw - 1) // 2)

    def _forward_direct(self, s, cell, filt):
        """The d-step forward on the direct correlation: each step's z from the (summed)
        previous state, then the non-fused epilogue (or port) with the hoisted border conv's
        delta as its border term (propagator.py:343-682)."""
        B, M, h, w, d = self.B, self.M, self.h, self.w, self.d
        kh, kw = self.kh, self.kw
        circ = int(self.circular)
        ws, nws = ptr(self.ws_epi), self.ws_epi.numel() * 4
        if self.border:  # propagator.py:362-366: conv_VALID(border patch, G)
            call("nc_direct_conv_fwd", s, 1, M, self.Hp, self.Wp, h, w, 0, 0, kh, kw, 0,
                 ptr(self.patch), 1, ptr(filt), ptr(self.delta))
        dl = ptr(self.delta) if self.border else None
        for t in range(d):
            z = self.zs[t if self.training else 0]
            x, n_parts, hin, win, oh, ow = self._conv_input(t)
            call("nc_direct_conv_fwd", s, B, M, hin, win, h, w, oh, ow, kh, kw, circ, ptr(x),
                 n_parts, ptr(filt), ptr(z))
            if t < d - 1:
                hb = int(self.border and t > 0)
                call("nc_epilogue_fwd_parts", s, B, M, h, w, self.act, self.slope, hb, ptr(z),
                     dl if hb else None, ptr(self.w_eff), ptr(self.s_eff), ptr(self.b_roi),
                     ptr(self.xs[t + 1]), ptr(self.mean[t]), ptr(self.rstd[t]), ws, nws)
                continue
            hb = int(self.border)
            if self.universe:
                call("nc_epilogue_fwd_parts", s, B, M, h, w, self.fact, self.fslope, hb, ptr(z),
                     dl if hb else None, ptr(self.w_eff), ptr(self.s_eff), ptr(self.b_roi),
                     ptr(self.port_parts), ptr(self.mean[t]), ptr(self.rstd[t]), ws, nws)
                call("nc_universe_fwd", s, self.chip, B, self.G, int(self.mode == "VALID"),
                     self.fact, self.fslope, ptr(self.port_parts), _addr(cell) + 4 * self.H *
                     self.W, ptr(self.s_prob), self.P, ptr(self.port_cells), ptr(self.univ),
                     ptr(self.out))
            elif self.dense_port:
                call("nc_epilogue_fwd_parts", s, B, M, h, w, self.fact, self.fslope, hb, ptr(z),
                     dl if hb else None, ptr(self.pp[0]), ptr(self.pp[1]), ptr(self.pp[2]),
                     ptr(self.port_parts), ptr(self.mean[t]), ptr(self.rstd[t]), ws, nws)
                call("nc_port_dense_fwd", s, B * self.P, self.G, self.fact, self.fslope,
                     ptr(self.port_parts), ptr(self.out), ptr(self.pre))
            else:
                call("nc_port_fwd", s, B, M, h, w, hb, self.fact, self.fslope, self.P,
                     ptr(self.port_idx), ptr(z), dl if hb else None, ptr(self.pp), ptr(self.out),
                     ptr(self.zo), ptr(self.mean[t]), ptr(self.rstd[t]), ptr(self.pre), ws, nws)
        return self.out

    def _backward_direct(self, s, cell, filt_used, g_out, g_cell, g_filt, codd, g_universe):
        """Reverse of _forward_direct: the port (or universe) backward, then per step the
        direct correlation's input and filter gradients and the epilogue backward, the border
        conv's reverse from the border cotangent, one sum of the filter-gradient rows."""
        B, M, h, w, d = self.B, self.M, self.h, self.w, self.d
        kh, kw, K = self.kh, self.kw, self.kh * self.kw
        circ = int(self.circular)
        ws, nws = ptr(self.ws_epi), self.ws_epi.numel() * 4
        valid = int(self.mode == "VALID")
        t = d - 1
        hb = int(self.border)
        dl = ptr(self.delta) if self.border else None
        gd = ptr(self.gdelta) if self.border else None
        params_written = False
        if self.universe:
            b_full = _addr(self.cell_s if self.sharpen is not None else cell) + 4 * self.H * self.W
            call("nc_universe_bwd", s, self.chip, B, self.G, valid, self.fact, self.fslope,
                 ptr(self.port_parts), b_full, ptr(self.s_prob), self.P, ptr(self.port_head),
                 ptr(self.port_next), ptr(g_out), ptr(g_universe), ptr(self.g_roi),
                 ptr(self.g_sprob) if valid else None, ptr(self.g_bfull) if valid else None)
            call("nc_epilogue_bwd", s, B, M, h, w, self.fact, self.fslope, hb, ptr(self.zs[t]),
                 dl if hb else None, ptr(self.w_eff), ptr(self.s_eff), ptr(self.b_roi),
                 ptr(self.mean[t]), ptr(self.rstd[t]), ptr(self.g_roi), ptr(self.gz),
                 gd if hb else None, ptr(self.gw), ptr(self.gs), ptr(self.gb), 0, 0, ws, nws)
            params_written = True
        elif self.dense_port:
            gy_port = g_out
            if self.fact != 0:
                call("nc_port_dense_bwd", s, B * self.P, self.fact, self.fslope, ptr(self.pre),
                     ptr(g_out), ptr(self.g_pre))
                gy_port = self.g_pre
            call("nc_epilogue_bwd", s, B, M, h, w, self.fact, self.fslope, hb, ptr(self.zs[t]),
                 dl if hb else None, ptr(self.pp[0]), ptr(self.pp[1]), ptr(self.pp[2]),
                 ptr(self.mean[t]), ptr(self.rstd[t]), ptr(gy_port), ptr(self.gz),
                 gd if hb else None, ptr(self.gpp[0]), ptr(self.gpp[1]), ptr(self.gpp[2]), 0, 0,
                 ws, nws)
        else:
            call("nc_port_bwd", s, B, M, h, w, hb, self.fact, self.fslope, self.P,
                 ptr(self.port_idx), ptr(self.zs[t]), dl if hb else None, ptr(self.pp),
                 ptr(self.zo), ptr(self.mean[t]), ptr(self.rstd[t]), ptr(self.pre), ptr(g_out),
                 ptr(self.gz), gd if hb else None, ptr(self.gpp) if self.n_pp else None, 0, ws,
                 nws)
        rows = _addr(self.dg_rows)
        step_bytes = 4 * self.dg_step_rows * M * K
        for t in range(d - 1, -1, -1):
            gy = self.gy[t % 2]
            x, n_parts, hin, win, oh, ow = self._conv_input(t)
            call("nc_direct_conv_bwd", s, B, M, hin, win, h, w, oh, ow, kh, kw, circ,
                 ptr(self.gz), ptr(x), n_parts, ptr(filt_used), int(t > 0),
                 ptr(gy) if t > 0 else None, rows + t * step_bytes)
            if t == 0:
                break
            te = t - 1
            hbe = int(self.border and te > 0)
            call("nc_epilogue_bwd", s, B, M, h, w, self.act, self.slope, hbe, ptr(self.zs[te]),
                 dl if hbe else None, ptr(self.w_eff), ptr(self.s_eff), ptr(self.b_roi),
                 ptr(self.mean[te]), ptr(self.rstd[te]), ptr(gy), ptr(self.gz),
                 gd if hbe else None, ptr(self.gw), ptr(self.gs), ptr(self.gb),
                 int(params_written), 1, ws, nws)
            params_written = True
        if self.border:  # the border conv's reverse: patch gradient and its filter rows
            call("nc_direct_conv_bwd", s, 1, M, self.Hp, self.Wp, h, w, 0, 0, kh, kw, 0,
                 ptr(self.gdelta), ptr(self.patch), 1, ptr(filt_used), 1, ptr(self.gpatch),
                 rows + d * step_bytes)
        call("nc_rows_sum", s, 1, _abi.rows_jobs((rows, _addr(g_filt), M * K, 0,
                                                  self.dg_rows.shape[0])))
        if self.gated:
            call("nc_filter_gate_bwd", s, self.filt_g.numel(), ptr(self.filt_g), ptr(g_filt))
        mode, inv_tau, active_threshold = codd
        sharp = self.sharpen is not None
        call("nc_codd_fuse_bwd", s, self.chip, ptr(self.cell_s if sharp else cell),
             ptr(self.io_mask), ptr(self.owm), mode, inv_tau, active_threshold,
             int(self.hard_pin_io), self.act, self.slope, self.n_pp, ptr(self.port_rc),
             *self._pp_csr(), ptr(self.gw) if params_written else None,
             ptr(self.gs) if params_written else None, ptr(self.gb) if params_written else None,
             ptr(self.gpatch) if self.border else None, ptr(self.gpp) if self.n_pp else None,
             ptr(self.g_sprob) if self.universe and valid else None,
             ptr(self.g_bfull) if self.universe and valid else None,
             ptr(self.g_cell_s if sharp else g_cell))
        if sharp:
            self._sharpen_bwd(s, g_cell)

    def _pp_csr(self):
        """The port-by-cell lists for nc_codd_fuse_bwd (none without port parameters)."""
        return (ptr(self.pp_start), ptr(self.pp_list)) if self.n_pp else (None, None)

    def _sharpen_bwd(self, s, g_cell):
        """The sharpening's adjoint on the weights' gradient."""
        ks = self.sharpen.shape
        g_cell[1:].copy_(self.g_cell_s[1:])
        call("nc_fftconv_bwd", s, 1, 1, self.H, self.W, self.H, self.W, (ks[0] - 1) // 2,
             (ks[1] - 1) // 2, *self.sh_fft, ptr(self.g_cell_s[0]), ptr(self.sh_xhat),
             ptr(self.sh_ghat), 1, ptr(g_cell[0]), ptr(self.sh_dg), 0, 0, ptr(self.sh_ws),
             self.sh_ws.numel() * 4)

    # ------------------------------------------------------------------ reverse
    def backward(self, cell: torch.Tensor, filt: torch.Tensor, g_out: torch.Tensor | None,
                 g_cell: torch.Tensor, g_filt: torch.Tensor, codd_mode: str = "continuous",
                 inv_tau: float = 1.0, active_threshold: float = 0.6,
                 g_universe: torch.Tensor | None = None) -> None:
        """Reverse pass of the last ``forward``: writes g_cell (3,H,W) and g_filt (M,1,kh,kw).
        On the universe path ``g_universe`` (B,H,W) may add a cotangent on the final
        universe, and either cotangent may be None (zero)."""
        if not self.training:
            raise NeurocellError("plan was built for evaluation only")
        s = stream_ptr()
        if self.direct:
            return self._backward_direct(s, cell, self.filt_g if self.gated else filt, g_out,
                                         g_cell, g_filt, (_abi.CODD_IDS[codd_mode], inv_tau,
                                                          active_threshold), g_universe)
        B, M, h, w, d = self.B, self.M, self.h, self.w, self.d
        fh, fw = self.fft
        ws_ep, n_ep = ptr(self.ws_epi), self.ws_epi.numel() * 4
        ws_fc, n_fc = ptr(self.ws_fc), self.ws_fc.numel() * 4
        t = d - 1
        N, RN = h * w, self.R * h * w
        valid = int(self.mode == "VALID")
        if self.universe:
            b_full = _addr(self.cell_s if self.sharpen is not None else cell) + 4 * self.H * self.W
            call("nc_universe_bwd", s, self.chip, B, self.G, valid, self.fact, self.fslope,
                 ptr(self.port_parts), b_full, ptr(self.s_prob), self.P, ptr(self.port_head),
                 ptr(self.port_next), ptr(g_out), ptr(g_universe), ptr(self.g_roi),
                 ptr(self.g_sprob) if valid else None, ptr(self.g_bfull) if valid else None)
            call("nc_epilogue_bwd_parts", s, B, M, h, w, self.fact, self.fslope, 0,
                 ptr(self.zs[t]), None, ptr(self.w_eff), ptr(self.s_eff), ptr(self.b_roi),
                 ptr(self.mean[t]), ptr(self.rstd[t]), ptr(self.g_roi), ptr(self.gz),
                 _addr(self.pg_rows) + 4 * (d - 1) * RN, self.pg_rows[0].numel(), ws_ep, n_ep)
        elif self.dense_port:
            gy_port = g_out
            if self.fact != 0:
                call("nc_port_dense_bwd", s, B * self.P, self.fact, self.fslope, ptr(self.pre),
                     ptr(g_out), ptr(self.g_pre))
                gy_port = self.g_pre
            call("nc_epilogue_bwd_parts", s, B, M, h, w, self.fact, self.fslope, 0,
                 ptr(self.zs[t]), None, ptr(self.pp[0]), ptr(self.pp[1]), ptr(self.pp[2]),
                 ptr(self.mean[t]), ptr(self.rstd[t]), ptr(gy_port), ptr(self.gz),
                 ptr(self.pp_rows), self.pp_rows[0].numel(), ws_ep, n_ep)
        else:
            call("nc_port_bwd_parts", s, B, M, h, w, 0, self.fact, self.fslope, self.P,
                 ptr(self.port_idx), ptr(self.zs[t]), None, ptr(self.pp), ptr(self.zo),
                 ptr(self.mean[t]), ptr(self.rstd[t]), ptr(self.pre), ptr(g_out),
                 ptr(self.gz), ptr(self.pp_rows), B * self.P, ws_ep, n_ep)
        pg_plane = self.pg_rows[0].numel()
        valid_acc = 0
        gy_epi = None  # the cotangent of step t's output, whose epilogue reverse is pending
        for t in range(d - 1, -1, -1):
            gy = self.gy[t % 2]
            need_dx = int(t > 0)
            if t == 0 and self.t0_grid:  # VALID full-grid step: its own spectral shift
                if gy_epi is not None:
                    self._epilogue_bwd_parts(s, 0, gy_epi, RN, pg_plane, ws_ep, n_ep)
                r0, _, c0, _ = self.bbox
                call("nc_fftconv_bwd_parts", s, B, M, self.H, self.W, h, w, self.kh - 1 + r0,
                     self.kw - 1 + c0, fh, fw, ptr(self.gz), ptr(self.xhat[0]), ptr(self.ghat),
                     0, None, ptr(self.rows["dgv"]), 0, 0, None, 0, ws_fc, n_fc)
                valid_acc = 1
            else:
                # steps t >= 1 carried the border term: their cotangent's batch sum, summed
                # over those steps in the frequency domain, is the border conv's cotangent
                hbt = t > 0 and self.border
                tail = (ptr(self.xhat[t]), ptr(self.ghat), need_dx, ptr(gy) if need_dx else None,
                        ptr(self.rows["dg"]), int(t < d - 1), 0,
                        ptr(self.rows["gd"]) if hbt else None, int(t < d - 1))
                if gy_epi is None:  # the output step: gz came from the port's reverse
                    call("nc_fftconv_bwd_parts", s, B, M, h, w, h, w, self.cp[0], self.cp[1],
                         fh, fw, ptr(self.gz), *tail, ws_fc, n_fc)
                else:  # step t's epilogue reverse and its correlation reverse in one call
                    call("nc_epilogue_fftconv_bwd_parts", s, B, M, h, w, self.act, self.slope,
                         ptr(self.zs[t]), ptr(self.w_eff), ptr(self.s_eff), ptr(self.b_roi),
                         ptr(self.mean[t]), ptr(self.rstd[t]), ptr(gy_epi), ptr(self.gz),
                         _addr(self.pg_rows) + 4 * t * RN, pg_plane, h, w, self.cp[0],
                         self.cp[1], fh, fw, *tail, ws_ep, n_ep, ws_fc, n_fc)
            if t == 0:
                break
            gy_epi = gy  # step t - 1's epilogue reverse runs with the next correlation reverse
        only_t0_grid = self.t0_grid and d == 1
        # every row stack written above, summed in one launch
        jobs = []
        if self.npart > 1:
            keys = ([] if only_t0_grid else ["dg"]) + (["dgv"] if valid_acc else []) + \
                   (["gd"] if self.border else [])
            outs = {"dg": self.dghat, "dgv": self.dghat_v, "gd": self.gdelta_hat}
            jobs += [(_addr(self.rows[k]), _addr(outs[k]), 2 * M * self.F, 0, self.npart)
                     for k in keys]
        if self.n_epi > 0:
            jobs += [(_addr(self.pg_rows[i]), _addr(g), N, 0, self.n_epi * self.R)
                     for i, g in enumerate((self.gw, self.gs, self.gb))]
        if self.n_pp > 0:
            jobs += [(_addr(self.pp_rows[i]), _addr(self.gpp[i]), self.n_pp, 0,
                      self.pp_rows.shape[1]) for i in range(3)]
        if jobs:
            call("nc_rows_sum", s, len(jobs), _abi.rows_jobs(*jobs))
        g_patch = None
        if self.border:
            # the filter gradients and the border conv's reverse in one launch: the patch
            # gradient from the cotangent spectra (its dG came with the ROI steps' dghat,
            # through their border-shifted cell spectra)
            call("nc_filter_patch_bwd", s, M, self.kh, self.kw, fh, fw, self.cp[0], self.cp[1],
                 ptr(self.dghat), ptr(g_filt), 0, 0, self.Hp, self.Wp, self.kh - 1,
                 self.kw - 1, ptr(self.gdelta_hat), ptr(self.ghat), ptr(self.gpatch), ws_fc,
                 n_fc)
            g_patch = ptr(self.gpatch)
        elif not only_t0_grid:
            call("nc_filter_spectrum_bwd", s, M, self.kh, self.kw, fh, fw, self.cp[0],
                 self.cp[1], ptr(self.dghat), ptr(g_filt), 0, 0)
        if valid_acc:
            call("nc_filter_spectrum_bwd", s, M, self.kh, self.kw, fh, fw, self.kh - 1,
                 self.kw - 1, ptr(self.dghat_v), ptr(g_filt), int(not only_t0_grid), 0)
        if self.gated:  # the chain rule through the gate, in place
            call("nc_filter_gate_bwd", s, self.filt_g.numel(), ptr(self.filt_g), ptr(g_filt))
        has_epi = self.n_epi > 0
        mode = _abi.CODD_IDS[codd_mode]
        sharp = self.sharpen is not None
        call("nc_codd_fuse_bwd", s, self.chip, ptr(self.cell_s if sharp else cell),
             ptr(self.io_mask), ptr(self.owm), mode, inv_tau, active_threshold,
             int(self.hard_pin_io), self.act, self.slope, self.n_pp, ptr(self.port_rc),
             *self._pp_csr(), ptr(self.gw) if has_epi else None,
             ptr(self.gs) if has_epi else None, ptr(self.gb) if has_epi else None, g_patch,
             ptr(self.gpp) if self.n_pp else None,
             ptr(self.g_sprob) if self.universe and valid else None,
             ptr(self.g_bfull) if self.universe and valid else None,
             ptr(self.g_cell_s if sharp else g_cell))
        if sharp:
            self._sharpen_bwd(s, g_cell)

    def _epilogue_bwd_parts(self, s, te, gy, RN, pg_plane, ws_ep, n_ep):
        """Step te's hidden epilogue reverse into gz and its own R rows of the gw / gs / gb
        stacks."""
        B, M, h, w = self.B, self.M, self.h, self.w
        call("nc_epilogue_bwd_parts", s, B, M, h, w, self.act, self.slope, 0,
             ptr(self.zs[te]), None, ptr(self.w_eff), ptr(self.s_eff), ptr(self.b_roi),
             ptr(self.mean[te]), ptr(self.rstd[te]), ptr(gy), ptr(self.gz),
             _addr(self.pg_rows) + 4 * te * RN, pg_plane, ws_ep, n_ep)

    # ------------------------------------------------------------------ loss
    def mse(self, target: torch.Tensor, loss: torch.Tensor | None = None) -> torch.Tensor:
        """default_mse_loss (trainer.py:57-61) on the port outputs: writes the loss (into
        ``loss`` when given, a one-element device view) and g_out."""
        loss = self.loss if loss is None else loss
        call("nc_mse_loss", stream_ptr(), self.B * self.P, ptr(self.out), ptr(target),
             ptr(loss), ptr(self.g_out))
        return loss


def _addr(t: torch.Tensor) -> int:
    """Device address of a contiguous device tensor (for the ABI's job structs)."""
    return ptr(t).value


def _abi_int(name: str, *args) -> int:
    v = int(getattr(lib(), name)(*args))
    if v <= 0:
        raise NeurocellError(f"{name}{args} failed")
    return v


def _abi_size(name: str, *args) -> int:
    from ._lib import lib
    return int(getattr(lib(), name)(*args))


def inv_tau_f32(state_temperature: float) -> float:
    """1 / max(tau, 1e-4) evaluated in float32 (params.py:63)."""
    t = np.float32(max(np.float32(state_temperature), np.float32(1e-4)))
    return float(np.float32(1.0) / t)


class ParamState:
    """Flat fp32 parameters (cell_params (3,H,W) then greens_filters (M,1,kh,kw)), their
    gradient and the AdamW moments, shared by every train-step bucket.  The step count and
    learning rate live in device memory so a captured step graph replays them."""

    def __init__(self, cell_params: torch.Tensor, filters: torch.Tensor,
                 learning_rate: float = 1e-3, b1: float = 0.9, b2: float = 0.999,
                 eps: float = 1e-8, weight_decay: float = 1e-4):
        dev = cell_params.device
        nc, nf = cell_params.numel(), filters.numel()
        self.n = nc + nf
        self.theta = torch.empty(self.n, device=dev, dtype=torch.float32)
        self.theta[:nc].copy_(cell_params.reshape(-1))
        self.theta[nc:].copy_(filters.reshape(-1))
        self.cell = self.theta[:nc].view(cell_params.shape)
        self.filt = self.theta[nc:].view(filters.shape)
        self.grad = torch.zeros_like(self.theta)
        self.g_cell = self.grad[:nc].view(cell_params.shape)
        self.g_filt = self.grad[nc:].view(filters.shape)
        self.m = torch.zeros_like(self.theta)
        self.v = torch.zeros_like(self.theta)
        self.count = torch.zeros(1, device=dev, dtype=torch.int32)
        self.set_learning_rate(learning_rate)
        self.hyper = (float(b1), float(b2), float(eps), float(weight_decay))

    def set_learning_rate(self, learning_rate) -> None:
        """A float, or a device/host table of the schedule at steps 0..n-1 (the last entry
        holds for later steps).  Replacing the table invalidates captured graphs."""
        t = torch.as_tensor(learning_rate, dtype=torch.float32).reshape(-1)
        self.lr = t.to(self.theta.device).contiguous()

    def adamw(self) -> None:
        b1, b2, eps, wd = self.hyper
        call("nc_adamw_step", stream_ptr(), self.n, ptr(self.theta), ptr(self.grad), ptr(self.m),
             ptr(self.v), ptr(self.count), ptr(self.lr), self.lr.numel(), b1, b2, eps, wd)


class TrainState:
    """One optimiser step of VNNTrainer.train_step (trainer.py:101-106) on a StepPlan:
    forward -> MSE loss -> reverse pass -> AdamW, over persistent buffers (static batch
    buffers ``x`` (B, n_in) and ``y`` (B, P)).  ``capture()`` records the whole step in a HIP
    graph that ``step()`` replays."""

    def __init__(self, plan: StepPlan, params: ParamState, codd_mode: str = "continuous",
                 state_temperature: float = 1.0, active_threshold: float = 0.6):
        self.plan = plan
        self.p = params
        dev = plan.device
        self.x = torch.zeros(plan.B, plan.n_in, device=dev, dtype=torch.float32)
        self.y = torch.zeros(plan.B, plan.P, device=dev, dtype=torch.float32)
        self.codd = (codd_mode, inv_tau_f32(state_temperature), float(active_threshold))
        self.graph = None

    def launch(self, x: torch.Tensor | None = None, y: torch.Tensor | None = None,
               loss: torch.Tensor | None = None) -> None:
        """Issues the step's launches on the current stream (no host synchronisation) for the
        batch ``x`` (B, n_in) / ``y`` (B, P), by default the static buffers."""
        pl, ps = self.plan, self.p
        mode, it, thr = self.codd
        pl.forward(ps.cell, ps.filt, self.x if x is None else x, codd_mode=mode, inv_tau=it,
                   active_threshold=thr)
        pl.mse(self.y if y is None else y, loss)
        pl.backward(ps.cell, ps.filt, pl.g_out, ps.g_cell, ps.g_filt, codd_mode=mode,
                    inv_tau=it, active_threshold=thr)
        ps.adamw()

    def capture(self) -> None:
        """Records one step into a HIP graph.  The warm-up launch on a side stream is a real
        optimiser step."""
        self.graph = _capture(self.launch)

    def step(self) -> torch.Tensor:
        if self.graph is not None:
            self.graph.replay()
        else:
            self.launch()
        return self.plan.loss


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


class EvalState:
    """Forward-only evaluation (VNNTrainer.evaluate_packed's apply, trainer.py:122-138) on an
    evaluation StepPlan, with optional HIP-graph capture."""

    def __init__(self, plan: StepPlan, cell_params: torch.Tensor, filters: torch.Tensor,
                 codd_mode: str = "continuous", state_temperature: float = 1.0,
                 active_threshold: float = 0.6):
        self.plan = plan
        self.cell = cell_params
        self.filt = filters
        self.x = torch.zeros(plan.B, plan.n_in, device=plan.device, dtype=torch.float32)
        self.codd = (codd_mode, inv_tau_f32(state_temperature), float(active_threshold))
        self.graph = None

    def launch(self) -> torch.Tensor:
        mode, it, thr = self.codd
        return self.plan.forward(self.cell, self.filt, self.x, codd_mode=mode, inv_tau=it,
                                 active_threshold=thr)

    def capture(self) -> None:
        self.graph = _capture(self.launch)

    def run(self) -> torch.Tensor:
        if self.graph is not None:
            self.graph.replay()
        else:
            self.launch()
        return self.plan.out

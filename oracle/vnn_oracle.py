"""CPU oracle for the Neurocell v2 VNN propagation step (float64 NumPy restatement).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or as the timed CPU baseline).  The product path under
``neurocell-v2_amd/`` never imports, links or calls anything under ``oracle/``.

Every function restates the reference's algorithm from its mathematics, citing
the reference file:line it follows (paths relative to the reference checkout).
The reference is JAX code that is not importable in this pipeline, so the
oracle is pinned instead by (see ``tests/test_oracle.py``):

* closed forms and known answers from the reference's own tests
  (ALU geometry, Codd-mode value sets, annealing end points, zero thresholding
  gap, factored == unfactored gating);
* brute force: direct spatial cross-correlation vs the FFT convolution, the
  full-grid legacy step vs the pure-ROI + hoisted-border decomposition;
* independent differentiation: every hand-written VJP is checked against
  central finite differences in float64 and against torch-CPU autograd of an
  independent restatement.

Parity pinned for every function in this file except ``adaptive_mask_stats``'s
salience thresholds, which are pinned only by the reference's frontier-growth
property test (no numeric golden exists; parity for the thresholds is
"partial").

Array conventions: NCHW, float64 unless ``dtype`` says otherwise.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

try:  # scipy's pocketfft honours ``workers``; numpy's FFT is the fallback
    import scipy.fft as _sfft

    def _rfft2(x, s, workers):
        return _sfft.rfft2(x, s=s, axes=(-2, -1), workers=workers)

    def _irfft2(x, s, workers):
        return _sfft.irfft2(x, s=s, axes=(-2, -1), workers=workers)
except ImportError:  # pragma: no cover
    def _rfft2(x, s, workers):
        return np.fft.rfft2(x, s=s, axes=(-2, -1))

    def _irfft2(x, s, workers):
        return np.fft.irfft2(x, s=s, axes=(-2, -1))

WORKERS = 1
_DTYPE = [np.float64]


def _dt():
    """Working float dtype (float64 for checking; float32 for the timed CPU baseline)."""
    return _DTYPE[0]


class precision:
    """``with precision(np.float32, workers=n):`` runs the oracle in float32 with n FFT
    workers (the CPU-baseline configuration)."""

    def __init__(self, dtype, workers=None):
        self.dtype, self.workers = dtype, workers

    def __enter__(self):
        global WORKERS
        self._saved = (_DTYPE[0], WORKERS)
        _DTYPE[0] = self.dtype
        if self.workers is not None:
            WORKERS = self.workers
        return self

    def __exit__(self, *exc):
        global WORKERS
        _DTYPE[0], WORKERS = self._saved

CODD_MODES = ("continuous", "annealed", "ste_binary", "ste_ternary")
EPS = 1e-5  # kernels_pallas.py:205 (rsqrt(var + 1e-5)), epilogue.py:25


# ---------------------------------------------------------------------------
# Activations — kernels_pallas.py:111-156
# ---------------------------------------------------------------------------

def act_fwd(x, name, neg_slope=0.01):
    """kernels_pallas.py:111-126."""
    if name in (None, "identity"):
        return x
    if name == "tanh":
        return np.tanh(x)
    if name == "sigmoid":
        return 1.0 / (1.0 + np.exp(-x))
    if name == "relu":
        return np.maximum(x, 0.0)
    if name == "leaky_relu":
        return np.where(x >= 0.0, x, neg_slope * x)
    if name == "gelu":
        c = math.sqrt(2.0 / math.pi)
        return 0.5 * x * (1.0 + np.tanh(c * (x + 0.044715 * x ** 3)))
    raise ValueError(name)


def act_deriv(x, name, neg_slope=0.01):
    """kernels_pallas.py:129-156 (derivative half)."""
    if name in (None, "identity"):
        return np.ones_like(x)
    if name == "tanh":
        y = np.tanh(x)
        return 1.0 - y * y
    if name == "sigmoid":
        y = 1.0 / (1.0 + np.exp(-x))
        return y * (1.0 - y)
    if name == "relu":
        return (x > 0.0).astype(x.dtype)
    if name == "leaky_relu":
        return np.where(x >= 0.0, 1.0, neg_slope).astype(x.dtype)
    if name == "gelu":
        c = math.sqrt(2.0 / math.pi)
        u = c * (x + 0.044715 * x ** 3)
        th = np.tanh(u)
        du = c * (1.0 + 3.0 * 0.044715 * x * x)
        return 0.5 * (1.0 + th) + 0.5 * x * (1.0 - th * th) * du
    raise ValueError(name)


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


# ---------------------------------------------------------------------------
# Geometry — topology.py:152-284 (VALID mode; the path's mode)
# ---------------------------------------------------------------------------

@dataclass
class Geometry:
    """Static chip geometry restated from ``ChipTopology2D.create`` (topology.py:152-284).

    ``in_ports``: list of ``("rect", (r0, c0), (h, w))`` or ``("coords", [(r, c), ...])``.
    ``out_port``: same encoding.
    """
    grid_shape: tuple
    kernel_size: tuple
    directions: int
    depth: int
    in_ports: list
    out_port: tuple
    pad_h: int = 0
    pad_w: int = 0
    roi_shape: tuple = (0, 0)
    fft_shape: tuple = (0, 0)
    io_state_mask: np.ndarray = field(default=None, repr=False)
    out_weight_mask: np.ndarray = field(default=None, repr=False)
    padding_mode: str = "VALID"

    def __post_init__(self):
        H, W = self.grid_shape
        kh, kw = self.kernel_size
        if kh % 2 == 0 or kw % 2 == 0:  # topology.py:174-175
            raise ValueError("kernel must be odd")
        self.padding_mode = self.padding_mode.upper()
        if self.padding_mode == "VALID":  # topology.py:184-189
            self.pad_h, self.pad_w = (kh - 1) // 2, (kw - 1) // 2
        else:
            self.pad_h, self.pad_w = 0, 0
        self.roi_shape = (H - 2 * self.pad_h, W - 2 * self.pad_w)  # :191-192
        npow2 = lambda v: 1 << (v - 1).bit_length()  # :89-91
        if self.padding_mode == "CIRCULAR":  # :256-258
            self.fft_shape = (H, W)
        else:
            self.fft_shape = (npow2(self.roi_shape[0] + kh - 1),
                              npow2(self.roi_shape[1] + kw - 1))
        io = np.zeros((H, W), bool)
        for p in self.in_ports:  # :238-245
            _mark(io, p)
        owm = np.zeros((H, W), bool)
        _mark(io, self.out_port)  # :248-254
        _mark(owm, self.out_port)
        self.io_state_mask, self.out_weight_mask = io, owm

    @property
    def out_cells_roi(self):
        """ROI-relative (rows, cols) of the output port cells in port order (row-major for rect)."""
        kind, a, *b = self.out_port
        if kind == "rect":
            (r0, c0), (h, w) = a, b[0]
            rows = [r0 + i for i in range(h) for j in range(w)]
            cols = [c0 + j for i in range(h) for j in range(w)]
        else:
            rows = [r for r, _ in a]
            cols = [c for _, c in a]
        return (np.asarray(rows) - self.pad_h, np.asarray(cols) - self.pad_w)

    @property
    def out_cells_grid(self):
        """Grid (rows, cols) of the output port cells in port order."""
        rows, cols = self.out_cells_roi
        return rows + self.pad_h, cols + self.pad_w

    @property
    def out_size(self):
        kind, a, *b = self.out_port
        return tuple(b[0]) if kind == "rect" else (len(a), 1)


def _mark(mask, port):
    kind, a, *b = port
    if kind == "rect":
        (r0, c0), (h, w) = a, b[0]
        mask[r0:r0 + h, c0:c0 + w] = True
    else:
        for r, c in a:
            mask[r, c] = True


def alu_geometry(n=8, kernel_size=(23, 13), directions=16, depth=4, gap=5, ctrl_gap=5,
                 out_width=1):
    """``ChipTopology2D.alu_chip`` restated (topology.py:286-321); ``out_width`` widens the
    output port column count (``out_width=2`` gives the 16-cell port of the benchmark configs)."""
    padding = 2 * max(kernel_size)
    N = 2 * n + padding
    center = N // 2
    input_top = center - (2 * n) // 2
    input_left = center - n
    output_mid = center - n // 2
    output_left = input_left + n + 2 * gap
    in_ports = [
        ("rect", (input_top, input_left), (n, 1)),
        ("rect", (input_top + n + 1, input_left), (n, 1)),
        ("rect", (input_top - ctrl_gap, input_left + gap), (1, n)),
    ]
    out_port = ("rect", (output_mid, output_left), (n, out_width))
    return Geometry((N, N), tuple(kernel_size), directions, depth, in_ports, out_port)


# ---------------------------------------------------------------------------
# Piece 1: Codd-state probabilities and the pre-step fusion
# ---------------------------------------------------------------------------

def inv_tau_f32(tau):
    """``1 / max(tau, 1e-4)`` evaluated in float32 as params.py:63 does."""
    t = np.float32(max(np.float32(tau), np.float32(1e-4)))
    return float(np.float32(1.0) / t)


def codd_state_probs(s_raw, io_mask, hard_pin_io=False, mode="continuous", tau=1.0,
                     active_threshold=0.6):
    """params.py:31-80.  Returns (s_prob, ds_prob/ds_raw) elementwise."""
    if mode not in CODD_MODES:
        raise ValueError(f"Unsupported codd_mode '{mode}'")
    s_raw = np.asarray(s_raw, dtype=_dt())
    s_base = s_raw if hard_pin_io else np.where(io_mask, 1.0, s_raw)
    if mode == "continuous":
        p = sigmoid(s_base)
        d = p * (1.0 - p)
    else:
        it = inv_tau_f32(tau)
        soft = sigmoid(s_base * it)
        d = it * soft * (1.0 - soft)
        if mode == "annealed":
            p = soft
        elif mode == "ste_binary":
            hard = np.where(s_base >= 0.0, 1.0, 0.0)
            p = soft + (hard - soft)
        else:
            hard = np.where(s_base >= active_threshold, 1.0, np.where(s_base > 0.0, 0.5, 0.0))
            p = soft + (hard - soft)
    if hard_pin_io:
        p = np.where(io_mask, 1.0, p)
    d = np.where(io_mask, 0.0, d)  # constant at pinned cells in both pin variants
    return p, d


def precompute_step_params(cell, geom: Geometry, act="tanh", hard_pin_io=False, roi_bbox=None,
                           mode="continuous", tau=1.0, active_threshold=0.6):
    """params.py:220-322.  ``cell`` is the (3,H,W) [W, B, S_raw] tensor."""
    H, W = geom.grid_shape
    rh, rw = geom.pad_h, geom.pad_w
    inv_M = 1.0 / float(geom.directions)
    w_raw, b_full, s_raw = (np.asarray(c, _dt()) for c in cell)
    w_pinned = np.where(geom.out_weight_mask, 1.0, w_raw)
    s_prob, ds = codd_state_probs(s_raw, geom.io_state_mask, hard_pin_io, mode, tau,
                                  active_threshold)
    roi = (slice(rh, H - rh), slice(rw, W - rw))
    w_roi, b_roi, s_roi = w_pinned[roi], b_full[roi], s_prob[roi]
    w_eff = inv_M * w_roi * (1.0 - s_roi)
    s_eff = inv_M * s_roi
    if roi_bbox is not None:
        r0, r1, c0, c1 = roi_bbox
        sub = (slice(r0, r1), slice(c0, c1))
    else:
        sub = (slice(None), slice(None))
    border_2d = act_fwd(b_full, act) * s_prob
    rows, cols = geom.out_cells_roi
    oh, ow = geom.out_size
    # port parameters exist for a port inside the ROI (a border port reads the universe)
    inside = (rows >= 0) & (rows < w_roi.shape[0]) & (cols >= 0) & (cols < w_roi.shape[1])
    rows, cols = np.where(inside, rows, 0), np.where(inside, cols, 0)
    port = lambda a: np.where(inside, a[rows, cols], 0.0).reshape(oh, ow)
    return dict(
        w_eff_roi=w_eff[sub], s_eff_roi=s_eff[sub], b_roi=b_roi[sub], border_2d=border_2d,
        w_eff_out=port(w_eff), s_eff_out=port(s_eff), b_out=port(b_roi),
        w_pinned=w_pinned, s_prob=s_prob, ds_prob=ds, b_full=b_full,
    )


def precompute_step_params_vjp(cell, geom: Geometry, grads: dict, act="tanh", hard_pin_io=False,
                               roi_bbox=None, mode="continuous", tau=1.0, active_threshold=0.6):
    """Reverse-mode derivative of :func:`precompute_step_params` (params.py:220-322 by hand).

    ``grads`` may hold ``w_eff_roi``, ``s_eff_roi``, ``b_roi`` (cropped shape), ``border_2d``,
    ``s_prob``, ``b_full`` (H, W), ``w_eff_out``, ``s_eff_out``, ``b_out`` (out_size).
    Returns g_cell (3, H, W).
    """
    H, W = geom.grid_shape
    rh, rw = geom.pad_h, geom.pad_w
    hv, wv = geom.roi_shape
    inv_M = 1.0 / float(geom.directions)
    sp = precompute_step_params(cell, geom, act, hard_pin_io, roi_bbox, mode, tau,
                                active_threshold)
    s_prob, ds = sp["s_prob"], sp["ds_prob"]
    b_full, w_pinned = sp["b_full"], sp["w_pinned"]
    g_weff = np.zeros((hv, wv), _dt())
    g_seff = np.zeros((hv, wv), _dt())
    g_broi = np.zeros((hv, wv), _dt())
    r0, r1, c0, c1 = roi_bbox if roi_bbox is not None else (0, hv, 0, wv)
    if "w_eff_roi" in grads:
        g_weff[r0:r1, c0:c1] += grads["w_eff_roi"]
    if "s_eff_roi" in grads:
        g_seff[r0:r1, c0:c1] += grads["s_eff_roi"]
    if "b_roi" in grads:
        g_broi[r0:r1, c0:c1] += grads["b_roi"]
    rows, cols = geom.out_cells_roi
    inside = (rows >= 0) & (rows < hv) & (cols >= 0) & (cols < wv)
    for key, dst in (("w_eff_out", g_weff), ("s_eff_out", g_seff), ("b_out", g_broi)):
        if key in grads:
            np.add.at(dst, (rows[inside], cols[inside]),
                      np.asarray(grads[key]).reshape(-1)[inside])
    roi = (slice(rh, H - rh), slice(rw, W - rw))
    g_wp = np.zeros((H, W), _dt())
    g_sp = np.zeros((H, W), _dt())
    g_b = np.zeros((H, W), _dt())
    s_roi = s_prob[roi]
    g_wp[roi] += inv_M * (1.0 - s_roi) * g_weff
    g_sp[roi] += -inv_M * w_pinned[roi] * g_weff + inv_M * g_seff
    g_b[roi] += g_broi
    if "border_2d" in grads:
        gbd = np.asarray(grads["border_2d"], _dt())
        g_b += act_deriv(b_full, act) * s_prob * gbd
        g_sp += act_fwd(b_full, act) * gbd
    if "s_prob" in grads:  # full-grid gradients on s_prob and on B themselves
        g_sp += np.asarray(grads["s_prob"], _dt())
    if "b_full" in grads:
        g_b += np.asarray(grads["b_full"], _dt())
    g_w = np.where(geom.out_weight_mask, 0.0, g_wp)
    g_s = g_sp * ds
    return np.stack([g_w, g_b, g_s])


# ---------------------------------------------------------------------------
# Input injection — propagator.py:88-100, 135-191
# ---------------------------------------------------------------------------

def inject_inputs_roi(port_inputs, geom: Geometry, roi_bbox=None):
    """``inject_inputs_roi_2d`` (propagator.py:135-191), including the per-port 3-D quirk:
    a (B, ih, iw) input is written with its OWN (ih, iw), not the declared port size.
    Returns (B, sub_h, sub_w) or raises if a port leaves the (cropped) ROI."""
    hv, wv = geom.roi_shape
    b_r0, b_r1, b_c0, b_c1 = roi_bbox if roi_bbox is not None else (0, hv, 0, wv)
    min_r, max_r = geom.pad_h + b_r0, geom.pad_h + b_r1
    min_c, max_c = geom.pad_w + b_c0, geom.pad_w + b_c1
    B = np.asarray(port_inputs[0]).shape[0]
    out = np.zeros((B, b_r1 - b_r0, b_c1 - b_c0), _dt())
    for inp, port in zip(port_inputs, geom.in_ports):
        inp = np.asarray(inp, _dt())
        kind, a, *b = port
        if kind == "coords":
            for k, (r, c) in enumerate(a):
                if not (min_r <= r < max_r and min_c <= c < max_c):
                    raise ValueError("port outside ROI")
                out[:, r - min_r, c - min_c] = inp.reshape(B, -1)[:, k]
            continue
        (r0, c0) = a
        if inp.ndim == 3:
            ih, iw = inp.shape[1], inp.shape[2]
            val = inp
        else:
            ih, iw = b[0]
            val = inp.reshape(B, ih, iw)
        if r0 < min_r or c0 < min_c or r0 + ih > max_r or c0 + iw > max_c:
            raise ValueError("port outside ROI")
        out[:, r0 - min_r:r0 - min_r + ih, c0 - min_c:c0 - min_c + iw] = val
    return out


def inject_inputs_full(port_inputs, geom: Geometry):
    """``inject_inputs_2d`` (propagator.py:103-132): the port inputs written into a zero
    (B, H, W) grid (a 3-D per-port input with its own (ih, iw))."""
    H, W = geom.grid_shape
    B = np.asarray(port_inputs[0]).shape[0]
    cells = np.zeros((B, H, W), _dt())
    for inp, port in zip(port_inputs, geom.in_ports):
        inp = np.asarray(inp, _dt())
        kind, a, *b = port
        if kind == "coords":
            for k, (r, c) in enumerate(a):
                cells[:, r, c] = inp.reshape(B, -1)[:, k]
            continue
        (r0, c0) = a
        ih, iw = inp.shape[1:] if inp.ndim == 3 else b[0]
        cells[:, r0:r0 + ih, c0:c0 + iw] = inp.reshape(B, ih, iw)
    return cells


def split_ports(inputs, geom: Geometry):
    """``_normalize_port_inputs`` (propagator.py:88-100)."""
    if isinstance(inputs, (list, tuple)):
        return list(inputs)
    inputs = np.asarray(inputs)
    if len(geom.in_ports) == 1:
        kind, a, *b = geom.in_ports[0]
        size = tuple(b[0]) if kind == "rect" else (len(a), 1)
        if inputs.ndim == 2 or (inputs.ndim == 3 and inputs.shape[1:] == size):
            return [inputs]
    return [inputs[:, i] for i in range(len(geom.in_ports))]


# ---------------------------------------------------------------------------
# Piece 2: Green's-function convolution (cross-correlation)
# ---------------------------------------------------------------------------

def conv2d_direct(x, g, pad):
    """Brute-force zero-padded cross-correlation, ``lax.conv_general_dilated`` semantics
    (kernels_greens.py:177-217): x (B,Hi,Wi), g (M,Kh,Kw), pad (ph,pw) -> (B,M,Ho,Wo)."""
    x = np.asarray(x, _dt())
    g = np.asarray(g, _dt())
    B, Hi, Wi = x.shape
    M, Kh, Kw = g.shape
    ph, pw = pad
    xp = np.zeros((B, Hi + 2 * ph, Wi + 2 * pw), _dt())
    xp[:, ph:ph + Hi, pw:pw + Wi] = x
    Ho, Wo = Hi + 2 * ph - Kh + 1, Wi + 2 * pw - Kw + 1
    out = np.zeros((B, M, Ho, Wo), _dt())
    for u in range(Kh):
        for v in range(Kw):
            out += xp[:, None, u:u + Ho, v:v + Wo] * g[None, :, u, v, None, None]
    return out


def filter_spectrum(g, fft_shape):
    """``precompute_filter_rfft2`` (kernels_greens.py:240-259): rfft2 of the flipped filters."""
    return _rfft2(np.flip(np.asarray(g, _dt()), axis=(-2, -1)), fft_shape, WORKERS)


def conv2d_fft(x, g, pad, out_shape, fft_shape):
    """Overlap-save spectral cross-correlation (kernels_greens.py:316-343, the forward of
    ``conv2d_roi_rfft_step``/``conv2d_pruned_rfft_roi_step``): z = irfft2(X * G_hat) cropped at
    ``pad``.  Also returns the cell spectrum X (the saved residual)."""
    fh, fw = fft_shape
    X = _rfft2(np.asarray(x), fft_shape, WORKERS)
    Gh = filter_spectrum(g, fft_shape)
    full = _irfft2(X[:, None] * Gh[None], fft_shape, WORKERS)
    (ho, wo), (r, c) = out_shape, pad
    # the window is read modulo the grid: the same slice where it fits, a circular
    # correlation where it wraps (the grid equal to the plane)
    full = np.roll(full, shift=(-r, -c), axis=(-2, -1))
    return full[..., :ho, :wo], X


def conv2d_circular_direct(x, g, pad):
    """CIRCULAR-mode step convolution as the reference writes it (propagator.py:284-292):
    the cells wrap-padded by ``pad`` (``jnp.pad(mode="wrap")``), then a brute-force VALID
    cross-correlation: x (B,H,W), g (M,Kh,Kw) -> (B,M,H,W)."""
    ph, pw = pad
    xp = np.pad(np.asarray(x, _dt()), ((0, 0), (ph, ph), (pw, pw)), mode="wrap")
    return conv2d_direct(xp, g, (0, 0))


def conv2d_fft_unshifted_bwd(gz, x, g, pad, fft_shape, need_dx=True):
    """Unshifted Plancherel backward (kernels_pallas.py:1794-1821 and :1558-1579):
    g_hat = rfft2(gz) at the origin; dx = irfft2(sum_m g_hat conj(G_hat)) rolled by ``pad``
    and cropped; dG_hat_unshifted = sum_b g_hat conj(X).  Returns (dx, dGhat_unshifted)."""
    B, Hi, Wi = np.asarray(x).shape
    X = _rfft2(np.asarray(x), fft_shape, WORKERS)
    Gh = filter_spectrum(g, fft_shape)
    gh = _rfft2(np.asarray(gz), fft_shape, WORKERS)
    dx = None
    if need_dx:
        full = _irfft2(np.sum(gh * np.conj(Gh)[None], axis=1), fft_shape, WORKERS)
        full = np.roll(full, shift=pad, axis=(-2, -1))
        dx = full[:, :Hi, :Wi]
    dGh = np.sum(gh * np.conj(X)[:, None], axis=0)
    return dx, dGh


def filter_grad_from_unshifted(dGh, kernel_size, pad, fft_shape):
    """``rfft2_unshifted_filter_grad_to_oihw`` (kernels_pallas.py:1558-1579) -> (M, Kh, Kw)."""
    kh, kw = kernel_size
    full = _irfft2(dGh, fft_shape, WORKERS)
    full = np.roll(full, shift=pad, axis=(-2, -1))
    return np.flip(full[:, :kh, :kw], axis=(-2, -1))


def conv2d_bwd_direct(gz, x, g, pad):
    """True gradient of :func:`conv2d_direct` by brute force: returns (dx, dg)."""
    gz = np.asarray(gz, _dt())
    x = np.asarray(x, _dt())
    g = np.asarray(g, _dt())
    B, Hi, Wi = x.shape
    M, Kh, Kw = g.shape
    ph, pw = pad
    Ho, Wo = gz.shape[-2:]
    xp = np.zeros((B, Hi + 2 * ph, Wi + 2 * pw), _dt())
    xp[:, ph:ph + Hi, pw:pw + Wi] = x
    dxp = np.zeros_like(xp)
    dg = np.zeros_like(g)
    for u in range(Kh):
        for v in range(Kw):
            dxp[:, u:u + Ho, v:v + Wo] += np.einsum("bmij,m->bij", gz, g[:, u, v])
            dg[:, u, v] = np.einsum("bmij,bij->m", gz, xp[:, u:u + Ho, v:v + Wo])
    return dxp[:, ph:ph + Hi, pw:pw + Wi], dg


# ---------------------------------------------------------------------------
# Piece 3: hidden-step epilogue and output-port epilogue
# ---------------------------------------------------------------------------

def standardize_stats(zt):
    """Two-pass population mean / rstd per (b, m) plane (kernels_pallas.py:202-205)."""
    mean = zt.mean(axis=(-2, -1))
    var = ((zt - mean[..., None, None]) ** 2).mean(axis=(-2, -1))
    return mean, 1.0 / np.sqrt(var + EPS)


def epilogue_fwd(z, delta, w, s, b, act="tanh", has_border=True, neg_slope=0.01):
    """``pallas_fused_roi_step_epilogue`` forward (kernels_pallas.py:163-218, 663-690;
    XLA twin epilogue.py:28-56).  Returns (out (B,Hv,Wv), mean (B,M), rstd (B,M))."""
    z = np.asarray(z, _dt())
    d = np.asarray(delta, _dt()).reshape((-1,) + z.shape[-3:])[0]
    zt = z + d[None] if has_border else z
    mean, rstd = standardize_stats(zt)
    zn = (zt - mean[..., None, None]) * rstd[..., None, None]
    out = w * zn.sum(1) + s * act_fwd(zn + b, act, neg_slope).sum(1)
    return out, mean, rstd


def epilogue_bwd(z, delta, w, s, b, mean, rstd, gy, act="tanh", has_border=True, neg_slope=0.01):
    """``_pallas_roi_epilogue_bwd_rule`` (kernels_pallas.py:221-291, 869-918).
    Returns (gz, gdb (M,Hv,Wv), gw, gs, gb)."""
    z = np.asarray(z, _dt())
    d = np.asarray(delta, _dt()).reshape((-1,) + z.shape[-3:])[0]
    zt = z + d[None] if has_border else z
    zn = (zt - mean[..., None, None]) * rstd[..., None, None]
    a = act_fwd(zn + b, act, neg_slope)
    da = act_deriv(zn + b, act, neg_slope)
    g_zn = gy[:, None] * (w + s * da)
    n = zn.shape[-1] * zn.shape[-2]
    c1 = g_zn.sum(axis=(-2, -1)) / n
    c2 = (g_zn * zn).sum(axis=(-2, -1)) / n
    gz = rstd[..., None, None] * (g_zn - c1[..., None, None] - zn * c2[..., None, None])
    gw = (gy * zn.sum(1)).sum(0)
    gs = (gy * a.sum(1)).sum(0)
    gb = (s * gy[:, None] * da).sum(axis=(0, 1))
    gdb = gz.sum(0) if has_border else np.zeros_like(d)
    return gz, gdb, gw, gs, gb


def port_fwd(z, delta, rows, cols, out_size, w_out, s_out, b_out, has_border=True,
             final_act=None):
    """``pallas_standardize_output_port`` + ``pallas_fused_output_port_epilogue``
    (kernels_pallas.py:1284-1347, 1510-1551; XLA twin epilogue.py:82-128).
    Returns (out (B,oh,ow), aux)."""
    z = np.asarray(z, _dt())
    d = np.asarray(delta, _dt()).reshape((-1,) + z.shape[-3:])[0]
    zt = z + d[None] if has_border else z
    mean, rstd = standardize_stats(zt)
    B, M = z.shape[:2]
    oh, ow = out_size
    zo = ((zt[:, :, rows, cols] - mean[..., None]) * rstd[..., None]).reshape(B, M, oh, ow)
    lin = zo.sum(1)
    if final_act is None:
        out = (w_out + s_out) * lin + float(M) * s_out * b_out
        pre = None
    else:
        pre = w_out * lin + s_out * act_fwd(zo + b_out, final_act).sum(1)
        out = act_fwd(pre, final_act)
    return out, dict(mean=mean, rstd=rstd, zo=zo, pre=pre)


def port_bwd(z, delta, rows, cols, out_size, w_out, s_out, b_out, aux, g_out, has_border=True,
             final_act=None):
    """Backward of :func:`port_fwd` (kernels_pallas.py:1350-1504 plus the jnp port algebra
    of :1538-1551).  Returns (gz, gdb, g_w_out, g_s_out, g_b_out)."""
    z = np.asarray(z, _dt())
    d = np.asarray(delta, _dt()).reshape((-1,) + z.shape[-3:])[0]
    zt = z + d[None] if has_border else z
    mean, rstd, zo = aux["mean"], aux["rstd"], aux["zo"]
    B, M = z.shape[:2]
    lin = zo.sum(1)
    if final_act is None:
        g_zo = np.broadcast_to((g_out * (w_out + s_out))[:, None], zo.shape)
        g_w = (g_out * lin).sum(0)
        g_s = (g_out * (lin + float(M) * b_out)).sum(0)
        g_b = (g_out * float(M) * s_out).sum(0)
    else:
        gp = g_out * act_deriv(aux["pre"], final_act)
        da = act_deriv(zo + b_out, final_act)
        g_zo = gp[:, None] * (w_out + s_out * da)
        g_w = (gp * lin).sum(0)
        g_s = (gp * act_fwd(zo + b_out, final_act).sum(1)).sum(0)
        g_b = (gp[:, None] * s_out * da).sum(axis=(0, 1))
    n = zt.shape[-1] * zt.shape[-2]
    g_flat = g_zo.reshape(B, M, -1)
    zo_flat = zo.reshape(B, M, -1)
    c1 = g_flat.sum(-1) / n
    c2 = (g_flat * zo_flat).sum(-1) / n
    zn = (zt - mean[..., None, None]) * rstd[..., None, None]
    gz = -rstd[..., None, None] * (c1[..., None, None] + zn * c2[..., None, None])
    for k, (r, c) in enumerate(zip(rows, cols)):
        gz[:, :, r, c] += rstd * g_flat[:, :, k]
    gdb = gz.sum(0) if has_border else np.zeros_like(d)
    return gz, gdb, g_w, g_s, g_b


# ---------------------------------------------------------------------------
# Orchestration — propagate_vnn_2d (propagator.py:209-682) and its VJP
# ---------------------------------------------------------------------------

def border_patch(border_2d, geom: Geometry, roi_bbox=None):
    """``border_only_2d`` (propagator.py:355-361): border_2d with the ROI zeroed, sliced to the
    cropped bbox's receptive field."""
    H, W = geom.grid_shape
    kh, kw = geom.kernel_size
    rh, rw = geom.pad_h, geom.pad_w
    bo = np.array(border_2d, _dt())
    bo[rh:H - rh, rw:W - rw] = 0.0
    if roi_bbox is not None:
        r0, r1, c0, c1 = roi_bbox
        bo = bo[r0:r1 + kh - 1, c0:c1 + kw - 1]
    return bo


def universe_embed(roi_final, sp, geom: Geometry, final_act=None, roi_bbox=None):
    """The final universe (propagator.py:700-731): the last step's sub-ROI epilogue output
    embedded in the grid, whose other cells hold final_act(B) * s_prob in VALID mode (zeros
    otherwise), then the final activation over the whole grid.  Returns (universe, pre)."""
    B = roi_final.shape[0]
    H, W = geom.grid_shape
    rh, rw = geom.pad_h, geom.pad_w
    hv, wv = geom.roi_shape
    r0, r1, c0, c1 = roi_bbox if roi_bbox is not None else (0, hv, 0, wv)
    if geom.padding_mode == "VALID":
        border = act_fwd(sp["b_full"], final_act) * sp["s_prob"]
    else:
        border = np.zeros((H, W), _dt())
    pre = np.broadcast_to(border, (B, H, W)).astype(_dt())
    pre[:, rh + r0:rh + r1, rw + c0:rw + c1] = roi_final
    return act_fwd(pre, final_act), pre


def universe_vjp(pre, g_out, g_universe, sp, geom: Geometry, final_act=None, roi_bbox=None):
    """Reverse of :func:`universe_embed` and the port read (the autodiff of
    propagator.py:700-734, :194-206): the port cotangents added at their cells, through the
    final activation onto the sub-ROI output (g_roi (B,h,w)) and, in VALID mode, the batch
    sum over the other cells onto s_prob and B (returned as the ``s_prob`` / ``b_full``
    gradients of :func:`precompute_step_params_vjp`)."""
    B, H, W = pre.shape
    g_fc = np.zeros((B, H, W), _dt()) if g_universe is None else np.array(g_universe, _dt())
    gr, gc = geom.out_cells_grid
    go = np.asarray(g_out, _dt()).reshape(B, -1)
    for p in range(go.shape[1]):
        g_fc[:, gr[p], gc[p]] += go[:, p]
    g_pre = g_fc * act_deriv(pre, final_act)
    rh, rw = geom.pad_h, geom.pad_w
    hv, wv = geom.roi_shape
    r0, r1, c0, c1 = roi_bbox if roi_bbox is not None else (0, hv, 0, wv)
    region = (slice(rh + r0, rh + r1), slice(rw + c0, rw + c1))
    extra = {}
    if geom.padding_mode == "VALID":
        gm = g_pre.sum(0)
        gm[region] = 0.0
        bf = sp["b_full"]
        extra = dict(s_prob=gm * act_fwd(bf, final_act),
                     b_full=gm * sp["s_prob"] * act_deriv(bf, final_act))
    return g_pre[:, region[0], region[1]], extra


def propagate(cell, filters, inputs, geom: Geometry, act="tanh", final_act=None,
              hard_pin_io=False, roi_bbox=None, mode="continuous", tau=1.0,
              active_threshold=0.6, conv="fft", universe=False):
    """Pure-ROI forward of ``propagate_vnn_2d`` for the pallas backends (propagator.py:252-682)
    and its CIRCULAR branch (:284-341); SAME and CIRCULAR have the whole grid as ROI and no
    border term.  ``filters`` is (M,1,Kh,Kw).  Returns (out, cache).  With ``universe`` the
    last step runs the full-grid output path (propagator.py:684-734): the port is read from the
    final universe, kept as ``cache["universe"]``."""
    valid = geom.padding_mode == "VALID"
    circular = geom.padding_mode == "CIRCULAR"
    if circular and roi_bbox is not None:
        raise ValueError("the CIRCULAR branch takes no sub-ROI")
    cell = np.asarray(cell, _dt())
    g = np.asarray(filters, _dt())[:, 0]
    kh, kw = geom.kernel_size
    pad = ((kh - 1) // 2, (kw - 1) // 2)
    d = geom.depth
    sp = precompute_step_params(cell, geom, act, hard_pin_io, roi_bbox, mode, tau,
                                active_threshold)
    try:
        x = inject_inputs_roi(split_ports(inputs, geom), geom, roi_bbox)
        t0_grid = False
        hv, wv = x.shape[-2:]
    except ValueError:
        # inputs outside the ROI: step 0 is the VALID correlation of the full injected grid
        # (propagator.py:347-352, 631-646)
        if not valid or roi_bbox is not None:
            raise
        x = inject_inputs_full(split_ports(inputs, geom), geom)
        t0_grid = True
        hv, wv = geom.roi_shape
    if roi_bbox is not None:
        fft_shape = (1 << (hv + kh - 2).bit_length(), 1 << (wv + kw - 2).bit_length())
    else:
        fft_shape = geom.fft_shape
    if valid:
        bp = border_patch(sp["border_2d"], geom, roi_bbox)
        delta = conv2d_direct(bp[None], g, (0, 0))[0]  # (M, hv, wv), propagator.py:362-366
    else:  # propagator.py:367-370
        bp = None
        delta = np.zeros((geom.directions, hv, wv), _dt())

    def _conv(xx):
        if conv == "direct":
            return conv2d_circular_direct(xx, g, pad) if circular else conv2d_direct(xx, g, pad)
        return conv2d_fft(xx, g, pad, (hv, wv), fft_shape)[0]

    xs, zs, stats = [x], [], []
    for t in range(d - 1):
        z = conv2d_direct(x, g, (0, 0)) if t == 0 and t0_grid else _conv(xs[-1])
        hb = t > 0 and valid
        out, mean, rstd = epilogue_fwd(z, delta, sp["w_eff_roi"], sp["s_eff_roi"], sp["b_roi"],
                                       act, hb)
        zs.append(z)
        stats.append((mean, rstd))
        xs.append(out)
    z = conv2d_direct(x, g, (0, 0)) if d == 1 and t0_grid else _conv(xs[-1])
    zs.append(z)
    rows, cols = geom.out_cells_roi
    if roi_bbox is not None:
        rows, cols = rows - roi_bbox[0], cols - roi_bbox[2]
    hb_final = d > 1 and valid
    univ = None
    if universe:
        roi_final, mean, rstd = epilogue_fwd(z, delta, sp["w_eff_roi"], sp["s_eff_roi"],
                                             sp["b_roi"], final_act, hb_final)
        univ, pre = universe_embed(roi_final, sp, geom, final_act, roi_bbox)
        gr, gc = geom.out_cells_grid
        out = univ[:, gr, gc].reshape((-1,) + tuple(geom.out_size))
        aux = dict(mean=mean, rstd=rstd, pre=pre)
    else:
        out, aux = port_fwd(z, delta, rows, cols, geom.out_size, sp["w_eff_out"],
                            sp["s_eff_out"], sp["b_out"], hb_final, final_act)
    cache = dict(sp=sp, xs=xs, zs=zs, stats=stats, delta=delta, bp=bp, aux=aux, g=g, pad=pad,
                 fft_shape=fft_shape, rows=rows, cols=cols, universe=univ, roi_bbox=roi_bbox,
                 t0_grid=t0_grid)
    return out, cache


def propagate_vjp(cell, filters, inputs, geom: Geometry, g_out, act="tanh", final_act=None,
                  hard_pin_io=False, roi_bbox=None, mode="continuous", tau=1.0,
                  active_threshold=0.6, fwd=None, universe=False, g_universe=None):
    """Reverse pass of :func:`propagate`: the chain of the reference's custom VJPs
    (kernels_pallas.py:1350-1504, 869-1064, 1794-1821, 1558-1579; propagator.py autodiff of
    the border conv and params.py autodiff of the pre-step fusion).
    ``fwd`` may pass the (out, cache) of a matching :func:`propagate` call to skip the
    forward.  With ``universe`` the cotangent is g_out on the port plus ``g_universe``
    (B,H,W, optional) on the final universe.  Returns (out, g_cell (3,H,W), g_filters
    (M,1,Kh,Kw))."""
    out, c = fwd if fwd is not None else propagate(
        cell, filters, inputs, geom, act, final_act, hard_pin_io, roi_bbox, mode, tau,
        active_threshold, universe=universe)
    sp, g, pad, fs = c["sp"], c["g"], c["pad"], c["fft_shape"]
    d = geom.depth
    kh, kw = geom.kernel_size
    M = geom.directions
    g_delta = np.zeros_like(c["delta"])
    g_weff = np.zeros_like(sp["w_eff_roi"])
    g_seff = np.zeros_like(sp["s_eff_roi"])
    g_broi = np.zeros_like(sp["b_roi"])
    valid = geom.padding_mode == "VALID"
    hb_final = d > 1 and valid
    extra = {}
    if c["universe"] is not None:
        aux = c["aux"]
        g_roi, extra = universe_vjp(aux["pre"], g_out, g_universe, sp, geom, final_act,
                                    roi_bbox)
        gz, gdb, gw, gs, gb = epilogue_bwd(c["zs"][-1], c["delta"], sp["w_eff_roi"],
                                           sp["s_eff_roi"], sp["b_roi"], aux["mean"],
                                           aux["rstd"], g_roi, final_act, hb_final)
        g_weff += gw
        g_seff += gs
        g_broi += gb
        g_wo = g_so = g_bo = np.zeros(geom.out_size, _dt())
    else:
        gz, gdb, g_wo, g_so, g_bo = port_bwd(c["zs"][-1], c["delta"], c["rows"], c["cols"],
                                             geom.out_size, sp["w_eff_out"], sp["s_eff_out"],
                                             sp["b_out"], c["aux"], np.asarray(g_out, _dt()),
                                             hb_final, final_act)
    g_delta += gdb
    dGh = np.zeros((M, fs[0], fs[1] // 2 + 1), complex)
    dg0 = 0.0
    for t in range(d - 1, -1, -1):
        x_t = c["xs"][t]
        if t == 0 and c["t0_grid"]:  # the full-grid VALID step's filter gradient
            dg0 = conv2d_bwd_direct(gz, x_t, g, (0, 0))[1]
            break
        dx, dG_t = conv2d_fft_unshifted_bwd(gz, x_t, g, pad, fs, need_dx=t > 0)
        dGh += dG_t
        if t == 0:
            break
        mean, rstd = c["stats"][t - 1]
        hb = (t - 1) > 0 and valid
        gz, gdb, gw, gs, gb = epilogue_bwd(c["zs"][t - 1], c["delta"], sp["w_eff_roi"],
                                           sp["s_eff_roi"], sp["b_roi"], mean, rstd, dx, act, hb)
        g_delta += gdb
        g_weff += gw
        g_seff += gs
        g_broi += gb
    g_filt = filter_grad_from_unshifted(dGh, (kh, kw), pad, fs) + dg0
    H, W = geom.grid_shape
    g_border = np.zeros((H, W), _dt())
    bp = c["bp"]
    if bp is not None:
        # border conv (1,1,Hp,Wp) VALID with G -> delta: adjoint by brute force
        Hp, Wp = bp.shape
        g_bp = np.zeros_like(bp)
        hv, wv = g_delta.shape[-2:]
        for u in range(kh):
            for v in range(kw):
                g_bp[u:u + hv, v:v + wv] += np.einsum("mij,m->ij", g_delta, g[:, u, v])
                g_filt[:, u, v] += np.einsum("mij,ij->m", g_delta, bp[u:u + hv, v:v + wv])
        r0, c0 = (roi_bbox[0], roi_bbox[2]) if roi_bbox is not None else (0, 0)
        g_border[r0:r0 + Hp, c0:c0 + Wp] = g_bp
        rh, rw = geom.pad_h, geom.pad_w
        g_border[rh:H - rh, rw:W - rw] = 0.0
    grads = dict(w_eff_roi=g_weff, s_eff_roi=g_seff, b_roi=g_broi, border_2d=g_border,
                 w_eff_out=g_wo, s_eff_out=g_so, b_out=g_bo, **extra)
    g_cell = precompute_step_params_vjp(cell, geom, grads, act, hard_pin_io, roi_bbox, mode,
                                        tau, active_threshold)
    return out, g_cell, g_filt[:, None]


def propagate_full_grid(cell, filters, inputs, geom: Geometry, act="tanh", final_act=None,
                        hard_pin_io=False, mode="continuous", tau=1.0, active_threshold=0.6,
                        return_universe=False):
    """Full-grid semantic definition (contrib/forward.py:737-810, driven as
    contrib/forward.py:162-178) using the v2 pinned/fused parameters: each step is a VALID
    correlation of the whole (B,H,W) grid, standardized, zero-padded back, Codd-gated and
    averaged over M.  Used to pin the pure-ROI + hoisted-border decomposition and the final
    universe (returned too with ``return_universe``)."""
    sp = precompute_step_params(cell, geom, act, hard_pin_io, None, mode, tau, active_threshold)
    g = np.asarray(filters, _dt())[:, 0]
    H, W = geom.grid_shape
    rh, rw = geom.pad_h, geom.pad_w
    M = geom.directions
    cells = inject_inputs_full(split_ports(inputs, geom), geom)
    B = cells.shape[0]
    w, bb, s = sp["w_pinned"], sp["b_full"], sp["s_prob"]

    def step(cells, a):
        zv = conv2d_direct(cells, g, (0, 0))
        mean, rstd = standardize_stats(zv)
        zn = (zv - mean[..., None, None]) * rstd[..., None, None]
        zp = np.zeros((B, M, H, W), _dt())
        zp[:, :, rh:H - rh, rw:W - rw] = zn
        lin = zp * w * (1.0 - s)
        nl = (zp + bb) * s if a is None else act_fwd(zp + bb, a) * s
        return (lin + nl).mean(1)

    for _ in range(geom.depth - 1):
        cells = step(cells, act)
    cells = step(cells, final_act)
    if final_act is not None:
        cells = act_fwd(cells, final_act)
    gr, gc = geom.out_cells_grid
    out = cells[:, gr, gc].reshape((B,) + tuple(geom.out_size))
    return (out, cells) if return_universe else out


# ---------------------------------------------------------------------------
# Piece 4: adaptive active-region bucketing — adaptive_mask.py
# ---------------------------------------------------------------------------

def quantize_interval(lo, hi, max_len, bucket_multiple):
    """``_quantize_interval`` (adaptive_mask.py:105-161), integer logic restated."""
    lo = max(0, min(lo, max_len - 1))
    hi = max(lo + 1, min(hi, max_len))
    raw = hi - lo
    if bucket_multiple <= 1 or raw >= max_len:
        return 0, max_len
    q = min(max_len, ((raw + bucket_multiple - 1) // bucket_multiple) * bucket_multiple)
    if q >= max_len or (max_len - q) < bucket_multiple:
        return 0, max_len
    ideal = lo - 0.5 * (q - raw)
    lo_min, lo_max = max(0, hi - q), min(lo, max_len - q)

    def best(step):
        first = ((lo_min + step - 1) // step) * step
        if first > lo_max:
            return None
        cands = range(first, lo_max + 1, step)
        return min(cands, key=lambda cc: (abs(cc - ideal), cc))

    new_lo = best(max(1, bucket_multiple // 2))
    if new_lo is None:
        new_lo = best(max(1, bucket_multiple // 4))
    if new_lo is None:
        new_lo = max(lo_min, min(int(round(ideal)), lo_max))
    return int(new_lo), int(new_lo + q)


def adaptive_mask_stats(cell, filters, io_mask_roi, geom: Geometry, margin=(4, 4),
                        salience_threshold=2.5, bias_threshold=0.05, filter_threshold=0.05,
                        act_roi=None, activity_threshold=1e-3):
    """``_compute_adaptive_mask_tensors`` (adaptive_mask.py:200-315): returns
    (stats int[8] = [r_eff_h, r_eff_w, salient, any_active, r0, r1, c0, c1], dilated mask)."""
    g = np.abs(np.asarray(filters, _dt())[:, 0])
    kh, kw = g.shape[-2:]
    mpt = g.max(0)
    active = mpt >= filter_threshold * mpt.max() + 1e-12
    rr = np.abs(np.arange(kh) - (kh - 1) // 2)[:, None]
    cc = np.abs(np.arange(kw) - (kw - 1) // 2)[None, :]
    r_eff_h = max(1, int(np.where(active, rr, 0).max()))
    r_eff_w = max(1, int(np.where(active, cc, 0).max()))
    H, W = geom.grid_shape
    rh, rw = geom.pad_h, geom.pad_w
    hv, wv = geom.roi_shape
    cell = np.asarray(cell, np.float32)
    w_roi = cell[0, rh:rh + hv, rw:rw + wv].astype(_dt())
    b_roi = cell[1, rh:rh + hv, rw:rw + wv].astype(_dt())
    s_roi = cell[2, rh:rh + hv, rw:rw + wv].astype(_dt())
    sp = sigmoid(s_roi)
    non_io = ~io_mask_roi
    non_io_count = max(1.0, float(non_io.sum()))
    drive = np.abs(b_roi) * sp
    upd = non_io & (np.abs(b_roi) > 1e-5)
    upd_count = max(1.0, float(upd.sum()))
    bm = np.where(upd, drive, 0.0).sum() / upd_count
    bs = math.sqrt(np.where(upd, (drive - bm) ** 2, 0.0).sum() / upd_count)
    zb = (drive - bm) / (bs + 1e-6)
    sal_b = non_io & (sp > 0.5) & (drive > bias_threshold) & (
        (zb > salience_threshold) | (drive > 4.0 * bias_threshold))
    wm = np.abs(w_roi) * sp
    wmean = np.where(non_io, wm, 0.0).sum() / non_io_count
    wstd = math.sqrt(np.where(non_io, (wm - wmean) ** 2, 0.0).sum() / non_io_count)
    zw = (wm - wmean) / (wstd + 1e-6)
    sal_r = non_io & (np.abs(b_roi) > 0.5 * bias_threshold) & (zw > salience_threshold) & (sp > 0.85)
    seed = io_mask_roi | sal_b | sal_r
    if act_roi is not None:
        seed = seed | (np.asarray(act_roi) > activity_threshold)
    mh, mw = margin
    dil = np.zeros_like(seed)
    for i in range(hv):
        for j in range(wv):
            dil[i, j] = seed[max(0, i - mh):i + mh + 1, max(0, j - mw):j + mw + 1].any()
    rows_any = dil.any(1)
    cols_any = dil.any(0)
    any_active = int(rows_any.any())
    r0 = int(np.where(rows_any, np.arange(hv), hv).min())
    r1 = int(np.where(rows_any, np.arange(hv), -1).max()) + 1
    c0 = int(np.where(cols_any, np.arange(wv), wv).min())
    c1 = int(np.where(cols_any, np.arange(wv), -1).max()) + 1
    return np.array([r_eff_h, r_eff_w, int(seed.sum()), any_active, r0, r1, c0, c1]), dil


# ---------------------------------------------------------------------------
# Trainer pieces — trainer.py:57-61, optax.adamw defaults
# ---------------------------------------------------------------------------

def mse_loss(logits, targets):
    """``default_mse_loss`` (trainer.py:57-61): mean squared error and its gradient."""
    logits = np.asarray(logits, _dt())
    targets = np.asarray(targets, _dt()).reshape(logits.shape)
    diff = logits - targets
    return float((diff ** 2).mean()), 2.0 * diff / diff.size


def adamw_step(p, g, m, v, count, lr, b1=0.9, b2=0.999, eps=1e-8, weight_decay=1e-4):
    """optax.adamw with default arguments (scale_by_adam -> add_decayed_weights ->
    scale_by_learning_rate), as the trainer's ``optax.adamw(lr)`` (trainer.py:101-106).
    Returns (p, m, v, count)."""
    count = count + 1
    m = b1 * m + (1.0 - b1) * g
    v = b2 * v + (1.0 - b2) * g * g
    mh = m / (1.0 - b1 ** count)
    vh = v / (1.0 - b2 ** count)
    u = mh / (np.sqrt(vh) + eps) + weight_decay * p
    return p - lr * u, m, v, count


def annealed_temperature(epoch, total_epochs, init_temp=1.0, final_temp=0.1,
                         schedule="exponential"):
    """``compute_annealed_temperature`` (trainer.py:23-46)."""
    if total_epochs <= 1:
        return float(final_temp)
    prog = min(1.0, max(0.0, float(epoch) / float(total_epochs - 1)))
    if schedule == "exponential":
        return float(init_temp * ((final_temp / init_temp) ** prog))
    if schedule == "cosine":
        return float(final_temp + (init_temp - final_temp) * 0.5 * (1.0 + math.cos(math.pi * prog)))
    if schedule == "linear":
        return float(init_temp + (final_temp - init_temp) * prog)
    raise ValueError(schedule)

"""Static chip geometry: ports, ROI bounds, FFT grid and pinning masks.

Host-side mirror of the reference's ``neurocell/topology.py`` (``PortSpec`` :19-34,
``CoordinatePortSpec`` :37-83, ``ChipTopology2D`` :109-284, ``alu_chip`` :286-321) with the
same constructor arguments, validation errors and derived fields.  Masks are NumPy ``bool``
arrays; device copies are made once by the step executor.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Sequence

import numpy as np


@dataclass(frozen=True)
class PortSpec:
    """Rectangular input/control/output port (topology.py:19-34)."""
    offset: tuple
    size: tuple
    name: str = ""

    def __post_init__(self):
        object.__setattr__(self, "offset", tuple(int(v) for v in self.offset))
        object.__setattr__(self, "size", tuple(int(v) for v in self.size))
        if len(self.offset) != len(self.size):
            raise ValueError(
                f"PortSpec offset {self.offset} and size {self.size} must have matching rank.")
        if any(s <= 0 for s in self.size):
            raise ValueError(f"PortSpec size dimensions must be positive, got {self.size}.")


@dataclass(frozen=True, init=False)
class CoordinatePortSpec:
    """Scattered (row, col) port (topology.py:37-83)."""
    coords: tuple
    name: str = ""

    def __init__(self, coords: Sequence[Sequence[int]], name: str = ""):
        coords_tuple = tuple((int(c[0]), int(c[1])) for c in coords)
        if len(coords_tuple) == 0:
            raise ValueError("CoordinatePortSpec coords must be non-empty.")
        object.__setattr__(self, "coords", coords_tuple)
        object.__setattr__(self, "name", str(name))

    @property
    def num_points(self) -> int:
        return len(self.coords)

    @property
    def size(self) -> tuple:
        return (len(self.coords), 1)

    @property
    def offset(self) -> tuple:
        return (min(r for r, _ in self.coords), min(c for _, c in self.coords))

    @property
    def rows(self) -> np.ndarray:
        return np.array([r for r, _ in self.coords], dtype=np.int32)

    @property
    def cols(self) -> np.ndarray:
        return np.array([c for _, c in self.coords], dtype=np.int32)

    def fits_in_roi(self, grid_shape, r_h, r_w) -> bool:
        H, W = grid_shape
        return all(r_h <= r < H - r_h and r_w <= c < W - r_w for r, c in self.coords)


def _next_power_of_two(x: int) -> int:
    return 1 << (int(x) - 1).bit_length()


def _port_within_bounds(port, r_min, r_max, c_min, c_max) -> bool:
    if isinstance(port, CoordinatePortSpec):
        return all(r_min <= r < r_max and c_min <= c < c_max for r, c in port.coords)
    r0, c0 = port.offset
    rh, cw = port.size
    return r0 >= r_min and c0 >= c_min and r0 + rh <= r_max and c0 + cw <= c_max


@dataclass(frozen=True)
class ChipTopology2D:
    """Immutable chip geometry (topology.py:109-284)."""
    grid_shape: tuple
    kernel_size: tuple
    directions: int
    depth: int
    in_ports: tuple
    out_port: object
    pad_h: int
    pad_w: int
    roi_shape: tuple
    roi_out_offset: tuple
    io_state_mask: np.ndarray = field(repr=False, compare=False)
    out_weight_mask: np.ndarray = field(repr=False, compare=False)
    fft_shape: tuple = (64, 64)
    padding_mode: str = "VALID"
    in_in_roi: bool = True
    out_in_roi: bool = True

    def __hash__(self):
        return hash((self.grid_shape, self.kernel_size, self.directions, self.depth,
                     self.in_ports, self.out_port, self.roi_shape, self.roi_out_offset,
                     self.fft_shape, self.padding_mode))

    @property
    def H(self) -> int:
        return self.grid_shape[0]

    @property
    def W(self) -> int:
        return self.grid_shape[1]

    @property
    def N(self) -> int:
        return max(self.grid_shape)

    @classmethod
    def create(cls, grid_shape, kernel_size, directions, depth, in_ports, out_port,
               fft_shape=None, padding_mode="VALID", allow_border_output=False):
        """topology.py:152-284, same validation and derived fields."""
        if isinstance(grid_shape, int):
            grid_shape = (grid_shape, grid_shape)
        else:
            grid_shape = (int(grid_shape[0]), int(grid_shape[1]))
        kh, kw = int(kernel_size[0]), int(kernel_size[1])
        if kh % 2 == 0 or kw % 2 == 0:
            raise ValueError(f"Green's function kernel_size must be odd, got {kernel_size}.")
        padding_mode = padding_mode.upper()
        if padding_mode not in ("VALID", "SAME", "CIRCULAR"):
            raise ValueError(f"Unsupported padding_mode '{padding_mode}'; choose from "
                             "('VALID', 'SAME', 'CIRCULAR').")
        H, W = grid_shape
        pad_h, pad_w = ((kh - 1) // 2, (kw - 1) // 2) if padding_mode == "VALID" else (0, 0)
        roi_h, roi_w = H - 2 * pad_h, W - 2 * pad_w
        if roi_h <= 0 or roi_w <= 0:
            raise ValueError(f"Grid {grid_shape} is too small for kernel {kernel_size}; "
                             f"valid ROI is ({roi_h}, {roi_w}).")
        in_ports = tuple(in_ports)
        for port in in_ports + (out_port,):
            if not _port_within_bounds(port, 0, H, 0, W):
                raise ValueError(f"Port '{port.name}' at offset={port.offset}, size={port.size} "
                                 f"exceeds grid_shape={grid_shape}.")
        in_in_roi = all(_port_within_bounds(p, pad_h, H - pad_h, pad_w, W - pad_w)
                        for p in in_ports)
        out_in_roi = _port_within_bounds(out_port, pad_h, H - pad_h, pad_w, W - pad_w)
        is_full_grid_out = (isinstance(out_port, PortSpec) and out_port.offset == (0, 0)
                            and out_port.size == grid_shape)
        if (padding_mode == "VALID" and not out_in_roi and not allow_border_output
                and not is_full_grid_out):
            raise ValueError(f"Output port {out_port} lies outside the active VALID convolution "
                             f"ROI [{pad_h}:{H - pad_h}, {pad_w}:{W - pad_w}].")
        out_r, out_c = out_port.offset
        if isinstance(out_port, CoordinatePortSpec):
            roi_out_offset = (tuple(int(r - pad_h) for r, _ in out_port.coords),
                              tuple(int(c - pad_w) for _, c in out_port.coords))
        else:
            roi_out_offset = (max(0, out_r - pad_h), max(0, out_c - pad_w))
        io = np.zeros(grid_shape, bool)
        for port in in_ports:
            if isinstance(port, CoordinatePortSpec):
                io[port.rows, port.cols] = True
            else:
                (r0, c0), (rh, cw) = port.offset, port.size
                io[r0:r0 + rh, c0:c0 + cw] = True
        owm = np.zeros(grid_shape, bool)
        if isinstance(out_port, CoordinatePortSpec):
            io[out_port.rows, out_port.cols] = True
            owm[out_port.rows, out_port.cols] = True
        else:
            oh, ow = out_port.size
            io[out_r:out_r + oh, out_c:out_c + ow] = True
            owm[out_r:out_r + oh, out_c:out_c + ow] = True
        if fft_shape is None:
            if padding_mode == "CIRCULAR":
                fft_shape = (H, W)
            else:
                fft_shape = (_next_power_of_two(roi_h + kh - 1),
                             _next_power_of_two(roi_w + kw - 1))
        return cls(grid_shape=grid_shape, kernel_size=(kh, kw), directions=int(directions),
                   depth=int(depth), in_ports=in_ports, out_port=out_port, pad_h=pad_h,
                   pad_w=pad_w, roi_shape=(roi_h, roi_w), roi_out_offset=roi_out_offset,
                   io_state_mask=io, out_weight_mask=owm, fft_shape=tuple(fft_shape),
                   padding_mode=padding_mode, in_in_roi=in_in_roi, out_in_roi=out_in_roi)

    @classmethod
    def alu_chip(cls, n=8, kernel_size=(23, 13), directions=16, depth=4, gap=5, ctrl_gap=5,
                 out_width=1):
        """topology.py:286-321.  ``out_width`` (default 1 = the reference) widens the output
        port by extra columns; the benchmark configs use 2 (16 output cells)."""
        padding = 2 * max(kernel_size[0], kernel_size[1])
        N = 2 * n + padding
        center = N // 2
        input_top = center - (2 * n) // 2
        input_left = center - n
        output_mid = center - n // 2
        output_left = input_left + n + 2 * gap
        in_ports = (
            PortSpec(offset=(input_top, input_left), size=(n, 1), name="x1"),
            PortSpec(offset=(input_top + n + 1, input_left), size=(n, 1), name="x2"),
            PortSpec(offset=(input_top - ctrl_gap, input_left + gap), size=(1, n), name="ctrl"),
        )
        out_port = PortSpec(offset=(output_mid, output_left), size=(n, int(out_width)),
                            name="out")
        return cls.create(grid_shape=(N, N), kernel_size=kernel_size, directions=directions,
                          depth=depth, in_ports=in_ports, out_port=out_port)

    @classmethod
    def mlp_chip(cls, n=8, layers=5, ctrl_gap=1, kernel_size=(17, 3), directions=8):
        """topology.py:324-357: the vertical-MLP chip, one (3n + ctrl_gap) x 1 input column
        and an n x 1 output column 2*layers + 1 cells to its right (depth = that gap)."""
        N = 2 * n + 2 * max(kernel_size)
        mid = N // 2
        span = 2 * layers + 1
        in_h = 3 * n + ctrl_gap
        in_r, in_c = mid - in_h // 2, mid - span // 2
        out_c = in_c + span
        return cls.create(grid_shape=(N, N), kernel_size=kernel_size, directions=directions,
                          depth=out_c - in_c,
                          in_ports=(PortSpec(offset=(in_r, in_c), size=(in_h, 1), name="x_in"),),
                          out_port=PortSpec(offset=(mid - n // 2, out_c), size=(n, 1),
                                            name="out"))

    @classmethod
    def gol_chip(cls, grid_shape=(64, 64), kernel_size=(3, 3), directions=64, depth=2,
                 padding_mode="VALID", n=None):
        """topology.py:359-388: a full-grid cellular automaton; the input and output ports
        are the whole grid (allowed outside a VALID ROI)."""
        if n is not None:
            grid_shape = (int(n), int(n))
        elif isinstance(grid_shape, int):
            grid_shape = (grid_shape, grid_shape)
        grid_shape = tuple(int(v) for v in grid_shape)
        return cls.create(grid_shape=grid_shape, kernel_size=kernel_size, directions=directions,
                          depth=depth,
                          in_ports=(PortSpec(offset=(0, 0), size=grid_shape,
                                             name="universe_in"),),
                          out_port=PortSpec(offset=(0, 0), size=grid_shape,
                                            name="universe_out"),
                          padding_mode=padding_mode, allow_border_output=True)

    @classmethod
    def clp_chip(cls, grid_shape=(8, 8), in_coords=None, out_coords=None, kernel_size=(3, 3),
                 directions=1, depth=4, padding_mode="VALID", n=None):
        """topology.py:390-428: the coordinate-addressed circular layered perceptron; by
        default two inputs one cell inside the left edge of the ROI and two outputs one cell
        inside its right edge (top and bottom rows)."""
        if n is not None:
            grid_shape = (int(n), int(n))
        elif isinstance(grid_shape, int):
            grid_shape = (grid_shape, grid_shape)
        H, W = (int(v) for v in grid_shape)
        valid = padding_mode.upper() == "VALID"
        rh = (kernel_size[0] - 1) // 2 if valid else 0
        rw = (kernel_size[1] - 1) // 2 if valid else 0
        top, bottom, left, right = rh + 1, H - rh - 2, rw + 1, W - rw - 2
        if in_coords is None:
            in_coords = ((top, left), (bottom, left))
        if out_coords is None:
            out_coords = ((top, right), (bottom, right))
        return cls.create(grid_shape=(H, W), kernel_size=kernel_size, directions=directions,
                          depth=depth, in_ports=(CoordinatePortSpec(in_coords, name="clp_in"),),
                          out_port=CoordinatePortSpec(out_coords, name="clp_out"),
                          padding_mode=padding_mode, allow_border_output=True)

    @classmethod
    def tm_chip(cls, n=8, kernel_size=(13, 13), directions=16, gap=1):
        """topology.py:430-455: a Turing-machine tape, a 1 x 2n input row and a 1 x n output
        row gap cells after it on the centre row (depth = their column distance)."""
        pad = 2 * max(kernel_size)
        N = 2 * n + 2 * pad
        mid = N // 2
        out_c = pad + 2 * n + gap
        return cls.create(grid_shape=(N, N), kernel_size=kernel_size, directions=directions,
                          depth=out_c - pad,
                          in_ports=(PortSpec(offset=(mid, pad), size=(1, 2 * n),
                                             name="tape_in"),),
                          out_port=PortSpec(offset=(mid, out_c), size=(1, n), name="tape_out"))

    def out_cells_grid(self) -> tuple:
        """Grid (rows, cols) int arrays of the output cells in port order (the cells
        _extract_output_from_full_grid reads, propagator.py:194-206)."""
        if isinstance(self.out_port, CoordinatePortSpec):
            return (np.asarray(self.out_port.rows, np.int32),
                    np.asarray(self.out_port.cols, np.int32))
        r0, c0 = self.out_port.offset
        oh, ow = self.out_port.size
        rr, cc = np.meshgrid(np.arange(oh), np.arange(ow), indexing="ij")
        return (r0 + rr.ravel()).astype(np.int32), (c0 + cc.ravel()).astype(np.int32)

    def out_cells_roi(self) -> tuple:
        """ROI-relative (rows, cols) int arrays of the output cells in port order."""
        if isinstance(self.out_port, CoordinatePortSpec):
            rows, cols = self.roi_out_offset
            return np.asarray(rows, np.int32), np.asarray(cols, np.int32)
        ro_r, ro_c = self.roi_out_offset
        oh, ow = self.out_port.size
        rr, cc = np.meshgrid(np.arange(oh), np.arange(ow), indexing="ij")
        return (ro_r + rr.ravel()).astype(np.int32), (ro_c + cc.ravel()).astype(np.int32)

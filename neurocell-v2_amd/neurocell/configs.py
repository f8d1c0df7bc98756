"""The five benchmark workloads of the MI355X build as data: chip geometry, ports, batch, Codd
mode and the seeded synthetic inputs and parameters.  ``bench.py`` and the parity tests build
their topologies and inputs from here, so both run the same shapes.

Parameters follow one distribution for every config: W ~ N(0, 0.1), bias ~ N(0, 0.01),
Codd logits S ~ N(0, 1) on (3, H, W), Green's filters ~ N(0, 1/K) read as variance 1/K with
K = kh*kw.  Targets are seeded random bits on the output port.

* config 0 -- 62x62 ALU chip (topology.py:286-321, output port widened to 8x2 = 16 cells),
  K = 23x13, M = 16, d = 4, B = 128, continuous; inputs are two uniform 8-bit operands and a
  3-bit opcode written as {0,1} cells (the ctrl operand as an 8x1 column, as the reference ALU
  driver does).  One train step.
* config 1 -- the same chip, forward-only evaluation at B = 1024, ste_ternary at tau = 0.1,
  uniform random port bits.
* config 2 -- large receptive field: K = 63x63 on a 174x174 VALID grid, so the ROI is
  112x112 (12,544 cells, the tiled epilogue) and the spectral grid 256x256; M = 16, d = 8,
  B = 64, annealed at tau = 0.1; 32 input cells (a 32x1 port) with uniform {0,1} values.
  The literal 128x128 grid with K = 63 has only a 66x66 ROI; ``config2_literal`` keeps it
  (spectral grid 128x128).
* config 3 -- 256x256 grid, K = 31x31, M = 32, d = 8, B = 32, continuous, with the active
  region cropped to 224x224 = 49 x 1024 cells (roi_bbox (1, 225, 1, 225) inside the 226x226
  VALID ROI; spectral grid 256x256); inputs N(0,1) on a 64-cell band (a 64x1 port).
* config 4 -- the ALU chip with the active region cropped to 24x32 (roi_bbox (6, 30, 10, 42),
  ROI rows 7..28 hold every port), B = 512, ste_binary at tau = 0.1.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .topology import ChipTopology2D, PortSpec


@dataclass(frozen=True)
class BenchConfig:
    name: str
    grid: tuple
    kernel: tuple
    directions: int
    depth: int
    batch: int
    codd_mode: str
    tau: float
    train: bool
    inputs: str            # "alu", "bits" or "normal"
    roi_bbox: tuple | None = None
    in_port: tuple | None = None   # (offset, size) of the single input port (non-ALU chips)
    out_port: tuple | None = None  # (offset, size) of the output port (non-ALU chips)

    def topology(self, depth: int | None = None, directions: int | None = None):
        d = self.depth if depth is None else depth
        m = self.directions if directions is None else directions
        if self.in_port is None:
            return ChipTopology2D.alu_chip(kernel_size=self.kernel, directions=m, depth=d,
                                           out_width=2)
        (ir, ic), isz = self.in_port
        (orr, oc), osz = self.out_port
        return ChipTopology2D.create(self.grid, self.kernel, m, d,
                                     in_ports=(PortSpec((ir, ic), isz, "in"),),
                                     out_port=PortSpec((orr, oc), osz, "out"))

    def synthetic(self, seed: int, batch: int | None = None, directions: int | None = None):
        """(cell_params (3,H,W), filters (M,1,kh,kw), inputs, targets) as float32 arrays."""
        B = self.batch if batch is None else batch
        M = self.directions if directions is None else directions
        rng = np.random.default_rng(seed)
        topo = self.topology(directions=M)
        H, W = topo.grid_shape
        kh, kw = self.kernel
        cell = np.stack([rng.normal(0, 0.1, (H, W)), rng.normal(0, 0.01, (H, W)),
                         rng.normal(0, 1.0, (H, W))]).astype(np.float32)
        filt = rng.normal(0, 1.0 / np.sqrt(kh * kw), (M, 1, kh, kw)).astype(np.float32)
        if self.inputs == "alu":
            a = rng.integers(0, 256, size=B, dtype=np.uint8)
            b = rng.integers(0, 256, size=B, dtype=np.uint8)
            op = rng.integers(0, 8, size=B, dtype=np.uint8)
            x = np.zeros((B, 3, 8, 1), np.float32)
            x[:, 0, :, 0] = np.unpackbits(a[:, None], axis=1)
            x[:, 1, :, 0] = np.unpackbits(b[:, None], axis=1)
            x[:, 2, :, 0] = np.unpackbits(op[:, None], axis=1)
        elif self.inputs == "bits":
            shape = (B, 3, 8, 1) if self.in_port is None else (B,) + tuple(self.in_port[1])
            x = rng.integers(0, 2, size=shape).astype(np.float32)
        else:
            x = rng.normal(size=(B,) + tuple(self.in_port[1])).astype(np.float32)
        y = rng.integers(0, 2, size=(B,) + tuple(topo.out_port.size)).astype(np.float32)
        return cell, filt, x, y


CONFIGS = {
    "config0": BenchConfig("config0", (62, 62), (23, 13), 16, 4, 128, "continuous", 1.0,
                           True, "alu"),
    "config1": BenchConfig("config1", (62, 62), (23, 13), 16, 4, 1024, "ste_ternary", 0.1,
                           False, "bits"),
    "config2": BenchConfig("config2", (174, 174), (63, 63), 16, 8, 64, "annealed", 0.1, True,
                           "bits", in_port=((71, 51), (32, 1)),
                           out_port=((83, 111), (8, 2))),
    "config2_literal": BenchConfig("config2_literal", (128, 128), (63, 63), 16, 8, 64,
                                   "annealed", 0.1, True, "bits",
                                   in_port=((40, 40), (32, 1)), out_port=((60, 80), (8, 2))),
    "config3": BenchConfig("config3", (256, 256), (31, 31), 32, 8, 32, "continuous", 1.0, True,
                           "normal", roi_bbox=(1, 225, 1, 225), in_port=((96, 56), (64, 1)),
                           out_port=((115, 195), (8, 2))),
    "config4": BenchConfig("config4", (62, 62), (23, 13), 16, 4, 512, "ste_binary", 0.1, True,
                           "alu", roi_bbox=(6, 30, 10, 42)),
}

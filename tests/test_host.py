"""CPU tests of the host side: the C ABI's exported symbols against the header, the product's
topology and bucketing logic against the reference's known answers and the oracle, the
trainer's schedules and helpers, parameter initialisation statistics, and the loud failure
of the product path without a device.  No kernel runs here."""
import ctypes
import math
import os
import re

import numpy as np
import pytest
import torch

from oracle import vnn_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "neurocell_hip.h")


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return dict(re.findall(r"^(?:int|size_t|const char\*)\s+(nc_\w+)\((.*?)\);", text,
                           flags=re.S | re.M))


def test_abi_table_matches_header():
    from neurocell import _abi
    funcs = _header_functions()
    assert set(funcs) == set(_abi.ENTRY_POINTS)
    for name, params in funcs.items():
        n = 0 if params.strip() == "void" else len([p for p in params.split(",") if p.strip()])
        assert len(_abi._SIGS[name][1]) == n, name


def test_library_exports_every_declared_symbol():
    from neurocell import _abi
    from neurocell._lib import lib_path
    if not os.path.exists(lib_path()):
        pytest.skip("native library not built")
    lib = ctypes.CDLL(lib_path())
    for name in _abi.ENTRY_POINTS:
        assert hasattr(lib, name), name
    lib = _abi.declare(lib)
    assert lib.nc_version() >= 1
    assert lib.nc_strerror(0) == b"ok"
    # workspace queries are pure host arithmetic
    assert lib.nc_epilogue_workspace_size(128, 16, 40, 50) > 0
    assert lib.nc_fftconv_bwd_workspace_size(128, 16, 64, 64) > 0


def test_fused_entry_queries_and_argument_checks():
    """Host arithmetic of the fused entries' partial counts and workspace sizes, and their
    argument checks (which return before any HIP call)."""
    from neurocell import _abi
    from neurocell._lib import lib_path
    if not os.path.exists(lib_path()):
        pytest.skip("native library not built")
    lib = _abi.declare(ctypes.CDLL(lib_path()))
    bad = _abi.NC_ERR_INVALID_ARGUMENT
    # the fused kernels run on the 32x64 / 64x64 grids: 4 directions per workgroup
    assert lib.nc_fftconv_epilogue_partials(128, 16, 40, 50, 64, 64) == 4
    assert lib.nc_fftconv_epilogue_partials(128, 6, 20, 27, 32, 64) == 2
    assert (lib.nc_fftconv_epilogue_partials(128, 16, 10, 12, 16, 16)
            == lib.nc_epilogue_fwd_partials(128, 16, 10, 12))
    epi = lib.nc_epilogue_workspace_size(1024, 64, 40, 50)
    assert lib.nc_fftconv_port_workspace_size(1024, 64, 40, 50, 64, 64, 256) == \
        max(epi, 2 * 16 * 1024 * 256 * 4)
    assert lib.nc_fftconv_port_workspace_size(8, 16, 10, 12, 16, 16, 16) == \
        lib.nc_epilogue_workspace_size(8, 16, 10, 12)
    # rejected before any launch
    assert lib.nc_fftconv_port_fwd(None, 2, 4, 40, 50, 11, 6, 64, 64, None, None, 0, 0.0, 0,
                                   None, None, None, None, None, None, None, None, None,
                                   0) == bad
    assert lib.nc_port_dense_fwd(None, 0, 1, 0, 0.0, None, None, None) == bad
    assert lib.nc_port_dense_bwd(None, 8, 0, 0.0, None, None, None) == bad
    assert lib.nc_filter_patch_bwd(None, 4, 5, 3, 16, 16, 2, 1, None, None, 0, 0, 17, 10, 4,
                                   2, None, None, None, None, 0) == bad
    assert lib.nc_fftconv_epilogue_fwd(None, 2, 4, 40, 50, 11, 6, 64, 64, None, None, 1, 0.0,
                                       None, None, None, None, None, None, None, None,
                                       0) == bad


def test_product_path_fails_loudly_without_device():
    if torch.cuda.is_available():
        pytest.skip("a device is visible")
    from neurocell import NeurocellError, VNNParams, propagate_vnn_2d
    from neurocell.topology import ChipTopology2D
    topo = ChipTopology2D.alu_chip()
    p = VNNParams(torch.zeros(3, 62, 62), torch.zeros(16, 1, 23, 13))
    with pytest.raises(NeurocellError):
        propagate_vnn_2d(p, torch.zeros(2, 3, 8, 1), topo)


# ------------------------------------------------------------------ topology

def test_topology_known_answers():
    """unit_topology.py:24-81."""
    from neurocell.topology import ChipTopology2D, PortSpec
    t = ChipTopology2D.alu_chip(n=8, kernel_size=(23, 13), directions=16, depth=4, gap=5,
                                ctrl_gap=5)
    assert t.grid_shape == (62, 62) and (t.H, t.W, t.N) == (62, 62, 62)
    assert (t.pad_h, t.pad_w) == (11, 6)
    assert t.roi_shape == (40, 50) and t.fft_shape == (64, 64)
    assert t.in_ports[0] == PortSpec(offset=(23, 23), size=(8, 1), name="x1")
    assert t.in_ports[1] == PortSpec(offset=(32, 23), size=(8, 1), name="x2")
    assert t.in_ports[2] == PortSpec(offset=(18, 28), size=(1, 8), name="ctrl")
    assert t.out_port == PortSpec(offset=(27, 41), size=(8, 1), name="out")
    assert t.roi_out_offset == (16, 35)
    assert int(t.io_state_mask.sum()) == 32 and int(t.out_weight_mask.sum()) == 8
    g = O.alu_geometry()
    assert np.array_equal(t.io_state_mask, g.io_state_mask)
    assert np.array_equal(t.out_weight_mask, g.out_weight_mask)
    with pytest.raises(ValueError):
        ChipTopology2D.create(grid_shape=(62, 62), kernel_size=(22, 13), directions=16, depth=4,
                              in_ports=(PortSpec((23, 23), (8, 1)),),
                              out_port=PortSpec((27, 41), (8, 1)))
    with pytest.raises(ValueError):
        ChipTopology2D.create(grid_shape=(62, 62), kernel_size=(23, 13), directions=16, depth=4,
                              in_ports=(PortSpec((23, 23), (8, 1)),),
                              out_port=PortSpec((2, 41), (8, 1)))


def test_out_cells_and_wide_port():
    from neurocell.topology import ChipTopology2D
    t = ChipTopology2D.alu_chip(out_width=2)
    rows, cols = t.out_cells_roi()
    g = O.alu_geometry(out_width=2)
    r2, c2 = g.out_cells_roi
    assert np.array_equal(rows, r2) and np.array_equal(cols, c2) and rows.size == 16


# ------------------------------------------------------------------ adaptive bucketing host logic

def test_quantize_interval_matches_oracle():
    from neurocell.adaptive_mask import _quantize_interval
    for max_len in (40, 50, 17):
        for bm in (1, 4, 8, 6):
            for lo in range(max_len):
                for hi in range(lo + 1, max_len + 1, 2):
                    assert _quantize_interval(lo, hi, max_len, bm) == \
                        O.quantize_interval(lo, hi, max_len, bm)


def test_cropped_topology():
    from neurocell.adaptive_mask import _build_cropped_topology
    from neurocell.topology import ChipTopology2D
    t = ChipTopology2D.alu_chip()
    c, fs = _build_cropped_topology(t, 2, 34, 10, 42)
    assert c.roi_shape == (32, 32) and c.roi_out_offset == (14, 25) and fs == (64, 64)
    c, fs = _build_cropped_topology(t, 6, 30, 10, 42)
    assert c.roi_shape == (24, 32) and fs == (64, 64)


def test_effective_filter_radii():
    """unit_milestone7_adaptive_mask.py:192-193: 3x3 filters give (1, 1)."""
    from neurocell import estimate_effective_filter_radii
    f = torch.randn(4, 1, 3, 3)
    assert estimate_effective_filter_radii(f) == (1, 1)
    g = torch.zeros(2, 1, 23, 13)
    g[0, 0, 11, 6] = 1.0
    g[1, 0, 11 + 7, 6 - 3] = 0.5
    assert estimate_effective_filter_radii(g) == (7, 3)


# ------------------------------------------------------------------ trainer host pieces

def test_annealed_temperature_endpoints():
    """unit_milestone8_pallas_and_codd.py:274-280."""
    from neurocell import compute_annealed_temperature as cat
    for sched in ("exponential", "cosine", "linear"):
        assert abs(cat(0, 10, 1.0, 0.1, sched) - 1.0) < 1e-9
        assert abs(cat(9, 10, 1.0, 0.1, sched) - 0.1) < 1e-9
        assert 0.1 < cat(5, 10, 1.0, 0.1, sched) < 1.0
        for e in range(10):
            assert cat(e, 10, 1.0, 0.1, sched) == O.annealed_temperature(e, 10, 1.0, 0.1, sched)
    with pytest.raises(ValueError):
        cat(0, 10, schedule="step")


def test_schedules_closed_forms():
    """optax schedule semantics: linear warmup then cosine decay to end_value
    (test_vnn_alu_arithmetic.py:172-178 parameters)."""
    from neurocell import warmup_cosine_decay_schedule, linear_schedule, cosine_decay_schedule
    total = 1000
    s = warmup_cosine_decay_schedule(0.001, 0.03, int(0.025 * total), total, 0.0005)
    assert s(0) == pytest.approx(0.001)
    assert s(25) == pytest.approx(0.03)
    assert s(12) == pytest.approx(0.001 + (0.03 - 0.001) * 12 / 25)
    assert s(total) == pytest.approx(0.0005) and s(10 * total) == pytest.approx(0.0005)
    mid = 25 + (total - 25) // 2
    frac = (mid - 25) / (total - 25)
    assert s(mid) == pytest.approx(0.0005 + (0.03 - 0.0005) * 0.5 * (1 + math.cos(math.pi * frac)))
    assert linear_schedule(1.0, 0.0, 0)(5) == 1.0
    with pytest.raises(ValueError):
        cosine_decay_schedule(1.0, 0)
    a = __import__("neurocell").adamw(s)
    tab = a.lr_table(30)
    assert tab.dtype == np.float32 and tab[0] == np.float32(0.001) and tab[25] == np.float32(0.03)


def test_packbits_and_losses():
    from neurocell import default_exact_match_metric, default_mse_loss, packbits_u8_on_device
    bits = torch.randint(0, 2, (5, 7, 8), dtype=torch.uint8)
    ref = np.packbits(bits.numpy(), axis=-1)
    assert np.array_equal(packbits_u8_on_device(bits).numpy(), ref)
    logits, y = torch.randn(4, 8, 1), torch.randn(4, 8)
    assert torch.allclose(default_mse_loss(logits, y), ((logits[..., 0] - y) ** 2).mean())
    t = torch.tensor([[0.5, 1.5, 2.5, -0.5]])
    assert float(default_exact_match_metric(t, torch.tensor([[0.0, 2.0, 2.0, 0.0]]))) == 1.0


def test_init_vnn_params_statistics():
    """params.py:145-217 distributions: truncated normals (|x| <= 2 sigma), sigmoid states,
    zero biases, pinned IO cells, OIHW filters."""
    from neurocell import init_vnn_params
    from neurocell.topology import ChipTopology2D
    t = ChipTopology2D.alu_chip()
    p = init_vnn_params(0, t, device="cpu")
    assert p.cell_params.shape == (3, 62, 62) and p.greens_filters.shape == (16, 1, 23, 13)
    w, b, s = p.cell_params
    io = torch.from_numpy(t.io_state_mask)
    assert torch.all(w[io] == 1.0) and torch.all(s[io] == 1.0) and torch.all(b == 0.0)
    std_w = math.sqrt((1.0 / math.sqrt(4 * 62)) / 62) / 0.87962566103423978
    wf = w[~io]
    assert float(wf.abs().max()) <= 2 * std_w + 1e-6
    assert abs(float(wf.std()) / (std_w * 0.87962566103423978) - 1.0) < 0.05
    sf = s[~io]
    assert float(sf.min()) > 0.0 and float(sf.max()) < 1.0
    std_f = math.sqrt((1.0 / math.sqrt(23 * 13 * 16)) / (23 * 13)) / 0.87962566103423978
    assert float(p.greens_filters.abs().max()) <= 2 * std_f + 1e-6
    q = init_vnn_params(0, t, device="cpu")
    assert torch.equal(p.cell_params, q.cell_params)


def test_checkpoint_roundtrip_cpu(tmp_path):
    from neurocell import VonNeumannNetwork, init_vnn_params
    from neurocell.topology import ChipTopology2D
    t = ChipTopology2D.alu_chip()
    m = VonNeumannNetwork(t)
    p = init_vnn_params(3, t, device="cpu")
    f = str(tmp_path / "c.npz")
    m.save_checkpoint(f, p, extra=np.int64(5))
    with np.load(f, allow_pickle=False) as d:
        assert d["filters"].shape == (1, 23, 13, 16) and int(d["N"]) == 62
        assert int(d["extra"]) == 5 and list(d["kernel_size"]) == [23, 13]
    q = VonNeumannNetwork.load_checkpoint(f, device="cpu")
    assert torch.equal(p.cell_params, q.cell_params)
    assert torch.equal(p.greens_filters, q.greens_filters)


def test_golden_checkpoint_loads():
    from neurocell import VonNeumannNetwork
    p = VonNeumannNetwork.load_checkpoint(os.path.join(ROOT, "tests/golden/alu_arithmetic_cells.npz"),
                                          device="cpu")
    assert p.cell_params.shape == (3, 62, 62) and p.greens_filters.shape == (16, 1, 23, 13)


def test_threshold_states():
    from neurocell import VonNeumannNetwork
    s = torch.tensor([-1.0, 0.0, 0.3, 0.6, 0.9])
    assert VonNeumannNetwork.threshold_states(s).tolist() == [-1.0, 0.0, 1.0, 2.0, 2.0]


def test_backend_selection_and_validation():
    from neurocell import SUPPORTED_BACKENDS, select_optimal_backend
    from neurocell.topology import ChipTopology2D
    assert SUPPORTED_BACKENDS == ("auto", "nchw_direct", "rfft_hoisted", "nchw_rfft_bwd",
                                  "pallas_fused", "pallas_sram")
    assert select_optimal_backend(ChipTopology2D.alu_chip()) == "pallas_fused"


@pytest.mark.parametrize("name", ["config0", "config1", "config2", "config2_literal", "config3",
                                  "config4"])
def test_benchmark_configs_geometry(name):
    """Each benchmark workload's topology agrees with the oracle's restatement of it, its ports
    lie inside the (cropped) ROI, and its spectral grid is one the C ABI covers."""
    from helpers import config_geometry
    from neurocell.configs import CONFIGS
    from neurocell.engine import spectral_grid_supported
    cfg = CONFIGS[name]
    topo, geom = cfg.topology(), config_geometry(cfg)
    assert topo.roi_shape == geom.roi_shape and tuple(topo.fft_shape) == geom.fft_shape
    assert (topo.io_state_mask == geom.io_state_mask).all()
    assert (topo.out_weight_mask == geom.out_weight_mask).all()
    rows, cols = topo.out_cells_roi()
    assert (rows == geom.out_cells_roi[0]).all() and (cols == geom.out_cells_roi[1]).all()
    r0, r1, c0, c1 = cfg.roi_bbox or (0, topo.roi_shape[0], 0, topo.roi_shape[1])
    assert rows.min() >= r0 and rows.max() < r1 and cols.min() >= c0 and cols.max() < c1
    kh, kw = cfg.kernel
    npow2 = lambda v: 1 << (v - 1).bit_length()
    fft = (npow2(r1 - r0 + kh - 1), npow2(c1 - c0 + kw - 1))
    assert spectral_grid_supported(*fft), fft
    expect = {"config0": (64, 64), "config1": (64, 64), "config2": (256, 256),
              "config2_literal": (128, 128), "config3": (256, 256), "config4": (64, 64)}
    assert fft == expect[name]
    cell, filt, x, y = cfg.synthetic(0, batch=2)
    assert cell.shape == (3,) + topo.grid_shape and filt.shape == (cfg.directions, 1) + cfg.kernel
    assert y.shape == (2,) + tuple(topo.out_port.size)


def test_chip_constructors_geometry():
    """topology.py:324-455: the MLP, Game-of-Life, CLP and Turing-machine chips."""
    from neurocell.topology import ChipTopology2D, CoordinatePortSpec
    m = ChipTopology2D.mlp_chip()  # n=8, 5 layers, K=17x3: N = 16 + 34
    assert m.grid_shape == (50, 50) and m.depth == 11
    assert m.in_ports[0].size == (25, 1) and m.out_port.size == (8, 1)
    assert m.out_port.offset[1] - m.in_ports[0].offset[1] == m.depth
    g = ChipTopology2D.gol_chip(n=32, padding_mode="SAME")
    assert g.grid_shape == (32, 32) and g.in_ports[0].size == (32, 32)
    assert g.out_port.size == (32, 32) and g.roi_shape == (32, 32)
    c = ChipTopology2D.clp_chip()
    assert isinstance(c.in_ports[0], CoordinatePortSpec)
    assert c.in_ports[0].coords == ((2, 2), (5, 2)) and c.out_port.coords == ((2, 5), (5, 5))
    cc = ChipTopology2D.clp_chip(n=16, padding_mode="CIRCULAR")
    assert cc.in_ports[0].coords == ((1, 1), (14, 1)) and cc.fft_shape == (16, 16)
    t = ChipTopology2D.tm_chip()  # n=8, K=13x13: N = 16 + 52
    assert t.grid_shape == (68, 68) and t.depth == 17
    assert t.in_ports[0].size == (1, 16) and t.out_port.offset == (34, 43)


def test_out_cells_grid_reads_ports_anywhere():
    """_extract_output_from_full_grid (propagator.py:194-206) reads the universe at the port's
    own grid cells: a rectangle on the border (VALID Game of Life) and coordinates."""
    from neurocell.topology import ChipTopology2D
    t = ChipTopology2D.gol_chip(n=6, kernel_size=(3, 3), directions=2, depth=2)
    assert not t.out_in_roi
    r, c = t.out_cells_grid()
    assert np.array_equal(r * 6 + c, np.arange(36))
    t = ChipTopology2D.clp_chip(n=8, out_coords=((0, 0), (7, 3), (4, 4)))
    r, c = t.out_cells_grid()
    assert r.tolist() == [0, 7, 4] and c.tolist() == [0, 3, 4]

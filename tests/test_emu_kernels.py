"""CPU parity of the kernel *sources*: the C ABI built with g++ against a CPU emulation of the
HIP device model (tests/emu), checked against the float64 oracle on small shapes.  These run
without a GPU; the same cases run on the MI355X in test_gpu_kernels.py."""
import ctypes

import pytest

from kernel_cases import (CODD_CASES, TOL, HostBackend, case_adaptive, case_border_conv,
                          case_border_fold, case_codd, case_epilogue, case_epilogue_parts,
                          case_fftconv_circular, case_fftconv_port, case_fftconv_epilogue,
                          case_fftconv, case_helpers, case_plane_spectra, case_port,
                          case_spectral_ops, case_direct_conv, case_epilogue_fftconv_bwd,
                          case_universe, case_fused_forms)


@pytest.fixture(scope="module")
def be():
    from emu.build_emu import build
    from neurocell import _abi
    return HostBackend(_abi.declare(ctypes.CDLL(build())))


def _assert_small(res, tol=TOL):
    bad = {k: v for k, v in res.items() if not v < tol}
    assert not bad, f"parity errors above {tol}: {bad} (all: {res})"


@pytest.mark.parametrize("FH,FW,hin,win,kh,kw", [
    (16, 16, 10, 12, 5, 3), (32, 64, 20, 50, 9, 13),
    (16, 64, 9, 40, 7, 13),     # FH < FW/2: the Nyquist staging spans fewer rows than lanes
    (64, 16, 50, 12, 13, 5),    # several row passes per wavefront (no LDS sharing)
    (64, 64, 41, 50, 23, 13),   # lane-pair transforms, odd row count (an unpaired row)
    (64, 64, 24, 32, 23, 13)])
def test_fftconv(be, FH, FW, hin, win, kh, kw):
    _assert_small(case_fftconv(be, B=2, M=3, hin=hin, win=win, kh=kh, kw=kw, FH=FH, FW=FW))


@pytest.mark.parametrize("B,M,FH,FW,hin,win,kh,kw", [
    (2, 3, 128, 128, 66, 60, 31, 21),     # one segment per pass
    (1, 2, 64, 256, 30, 150, 13, 63),     # asymmetric grids
    (2, 2, 256, 128, 150, 40, 63, 13),
    (1, 2, 256, 256, 224, 224, 31, 31),   # config-3 planes: two column and two row segments
    (2, 17, 128, 64, 40, 36, 9, 9)])      # two direction chunks in the backward reduction
def test_fftconv_large(be, B, M, FH, FW, hin, win, kh, kw):
    _assert_small(case_fftconv(be, B=B, M=M, hin=hin, win=win, kh=kh, kw=kw, FH=FH, FW=FW))


@pytest.mark.parametrize("FH,FW,h,w,kh,kw", [
    (32, 16, 12, 10, 7, 5),      # wavefront transforms (packed dx spectrum)
    (64, 64, 40, 50, 23, 13),    # lane-pair transforms
    (128, 64, 60, 30, 31, 13)])  # workgroup transforms
def test_border_conv(be, FH, FW, h, w, kh, kw):
    _assert_small(case_border_conv(be, h=h, w=w, kh=kh, kw=kw, FH=FH, FW=FW))


@pytest.mark.parametrize("FH,FW,h,w,kh,kw", [
    (32, 16, 12, 10, 7, 5), (64, 64, 40, 50, 23, 13), (128, 64, 60, 30, 31, 13)])
def test_border_fold(be, FH, FW, h, w, kh, kw):
    _assert_small(case_border_fold(be, h=h, w=w, kh=kh, kw=kw, FH=FH, FW=FW))


@pytest.mark.parametrize("FH,FW,h,w,kh,kw", [
    (32, 16, 12, 10, 7, 5), (64, 64, 40, 50, 23, 13), (128, 64, 60, 30, 31, 13)])
def test_plane_spectra(be, FH, FW, h, w, kh, kw):
    _assert_small(case_plane_spectra(be, h=h, w=w, kh=kh, kw=kw, FH=FH, FW=FW))


@pytest.mark.parametrize("shape", [(2, 3, 10, 12, "tanh", 1), (2, 3, 20, 40, "leaky_relu", 0),
                                   (1, 2, 96, 90, "gelu", 1), (1, 2, 91, 91, "tanh", 1),
                                   # directions split over workgroups (forward groups of 4,
                                   # backward groups of 8), the last group partial
                                   (3, 9, 10, 12, "tanh", 1), (2, 17, 6, 7, "sigmoid", 0)])
def test_epilogue(be, shape):
    _assert_small(case_epilogue(be, *shape))


@pytest.mark.parametrize("shape", [
    (2, 3, 10, 12, (2, 3, 4, 2), (5, 5, 5, 5), None),
    (3, 9, 10, 12, (2, 3, 4, 2), (5, 5, 5, 5), "tanh"),  # split port forward, ticket combine
    (1, 2, 96, 100, (10, 50, 95), (3, 99, 0), "tanh"),
    (2, 3, 12, 10, (1, 7, 7), (2, 3, 3), "sigmoid", 0)])  # no border term: gdb = 0
def test_port(be, shape):
    B, M, h, w, rows, cols, fact, *hb = shape
    _assert_small(case_port(be, B, M, h, w, rows, cols, fact, has_border=hb[0] if hb else 1))


@pytest.mark.parametrize("mode,bbox,hard_pin", CODD_CASES[::3])
def test_codd(be, mode, bbox, hard_pin):
    _assert_small(case_codd(be, mode, bbox, hard_pin), tol=1e-5)


def test_adaptive_stats(be):
    assert case_adaptive(be) == {"stats_mismatch": 0.0, "mask_mismatch": 0.0}


def test_helpers(be):
    res = case_helpers(be)
    assert res["inject_mismatch"] == 0 and res["count_mismatch"] == 0, res
    _assert_small({k: res[k] for k in ("mse", "g_mse", "adamw", "adamw_large")})


@pytest.mark.parametrize("B,M,h,w,FH,FW", [(3, 9, 10, 12, 16, 16), (2, 16, 40, 50, 64, 64)])
def test_epilogue_parts(be, B, M, h, w, FH, FW):
    res = case_epilogue_parts(be, B=B, M=M, h=h, w=w, kh=5, kw=3, FH=FH, FW=FW)
    assert res["G"] >= 1 and res["out"] < TOL, res
    assert res["parts_sum_mismatch"] == 0 and res["z_mismatch"] == 0, res
    assert res["xhat_mismatch"] == 0, res


@pytest.mark.parametrize("B,M,h,w,kh,kw,FH,FW,act,two_pass", [
    (3, 6, 20, 27, 7, 5, 32, 64, "tanh", False),          # fused, idle wavefronts
    (2, 16, 40, 50, 23, 13, 64, 64, "leaky_relu", False),  # fused, the ALU geometry
    (3, 5, 10, 12, 5, 3, 16, 16, "gelu", False),           # not fused: correlation + epilogue
    (2, 3, 60, 50, 31, 13, 128, 64, "tanh", True),     # two-pass large-grid correlation
    (1, 2, 224, 224, 31, 31, 256, 256, "tanh", True),  # config-3 planes, two passes
    (1, 3, 40, 150, 13, 63, 64, 256, "gelu", True),    # asymmetric grid, two passes
    (1, 3, 100, 100, 9, 9, 128, 128, "tanh", True),    # band statistics, 64-row bands
    (1, 2, 150, 80, 31, 13, 256, 128, "sigmoid", True),  # band statistics, 256 x 128 grid
])
def test_fftconv_epilogue(be, B, M, h, w, kh, kw, FH, FW, act, two_pass):
    res = case_fftconv_epilogue(be, B=B, M=M, h=h, w=w, kh=kh, kw=kw, FH=FH, FW=FW, act=act,
                                two_pass=two_pass)
    if FW == 64 and FH in (32, 64):
        assert res["G"] == (M + 3) // 4 and res["no_z_mismatch"] == 0, res
    assert res["xhat_mismatch"] == 0, res
    _assert_small({k: res[k] for k in ("z", "z_vs_separate", "out", "out_vs_separate", "mean",
                                       "rstd")})


def test_fused_forward_forms(be):
    """The fused forward's two forms agree to rounding, rel-L2 1e-6 (the emulated device has
    two CUs: one sample's four workgroups take the full-row form, three samples' twelve the
    windowed; their lanes sum the plane statistics in different pixel orders)."""
    res = case_fused_forms(be, 1, 3)
    assert res["forms"] < 1e-6 and res["z"] < TOL, res


@pytest.mark.parametrize("B,M,H,W,kh,kw", [
    (2, 3, 16, 16, 5, 3),     # wavefront transforms
    (2, 6, 32, 64, 7, 5),     # lane pairs, fused epilogue with idle wavefronts
    (2, 4, 64, 64, 9, 9),     # lane pairs + segmented per-sample transforms, 64 values/lane
    (1, 2, 128, 128, 5, 5),   # workgroup transforms over LDS segments
])
def test_fftconv_circular(be, B, M, H, W, kh, kw):
    res = case_fftconv_circular(be, B=B, M=M, H=H, W=W, kh=kh, kw=kw)
    _assert_small(res)


@pytest.mark.parametrize("B,M,h,w,kh,kw,FH,FW,fact,two_pass", [
    (3, 6, 20, 27, 7, 5, 32, 64, None, False),           # fused, idle wavefronts, identity port
    (2, 16, 40, 50, 23, 13, 64, 64, "tanh", False),      # fused, the ALU geometry, gated port
    (3, 5, 10, 12, 5, 3, 16, 16, "sigmoid", False),      # not fused: correlation then port
    (2, 3, 60, 50, 31, 13, 128, 64, "tanh", True),      # two-pass large-grid correlation
    (1, 2, 224, 224, 31, 31, 256, 256, None, True),
])
def test_fftconv_port(be, B, M, h, w, kh, kw, FH, FW, fact, two_pass):
    rows, cols = (2, 3, h - 1, 3, 0), (5, 5, w - 1, 5, 0)
    res = case_fftconv_port(be, B=B, M=M, h=h, w=w, kh=kh, kw=kw, FH=FH, FW=FW, fact=fact,
                            rows=rows, cols=cols, two_pass=two_pass)
    _assert_small(res)


UNIVERSE_CASES = [("VALID", None, "tanh"), ("VALID", (2, 9, 1, 10), "sigmoid"),
                  ("VALID", None, None), ("SAME", None, "relu"), ("SAME", (3, 12, 2, 11), "gelu")]


@pytest.mark.parametrize("pmode,bbox,fact", UNIVERSE_CASES)
def test_universe(be, pmode, bbox, fact):
    _assert_small(case_universe(be, pmode, bbox, fact))


@pytest.mark.parametrize("FH,FW,roi,pad,shift", [(32, 16, (12, 10), (5, 3), (7, 5)),
                                                 (64, 64, (40, 50), (11, 6), (63, 1))])
def test_spectral_ops(be, FH, FW, roi, pad, shift):
    _assert_small(case_spectral_ops(be, FH=FH, FW=FW, roi=roi, pad=pad, shift=shift))


@pytest.mark.parametrize("B,M,H,W,kh,kw,mode,n_parts", [
    (3, 5, 12, 14, 3, 3, "SAME", 2), (2, 4, 16, 16, 3, 3, "CIRCULAR", 1),
    (2, 3, 20, 18, 5, 3, "VALID", 1), (2, 16, 32, 32, 3, 3, "SAME", 4),
    (1, 2, 9, 40, 17, 3, "SAME", 1), (2, 3, 16, 16, 3, 5, "CIRCULAR", 2),
    (2, 1, 8, 8, 3, 3, "VALID", 1),          # one direction (a one-direction register tile)
    (1, 64, 12, 16, 7, 9, "SAME", 2),        # K = 63, M = 64: chunked cotangent staging
    (1, 3, 6, 200, 3, 5, "SAME", 1),         # a 200-wide plane: one row group per band
    (600, 2, 6, 6, 3, 3, "CIRCULAR", 1)])    # many samples: the smaller register tiles
def test_direct_conv(be, B, M, H, W, kh, kw, mode, n_parts):
    _assert_small(case_direct_conv(be, B, M, H, W, kh, kw, mode, n_parts))


@pytest.mark.parametrize("B,M,h,w,kh,kw,FH,FW,act", [
    (1, 2, 112, 112, 31, 21, 256, 256, "tanh"),   # fused: gz formed in the row pass
    (1, 2, 100, 100, 9, 9, 128, 128, "relu"),     # fused, 64-row bands
    (1, 2, 150, 82, 31, 13, 256, 128, "gelu"),    # fused, rows not a multiple of 4 wide
    (2, 3, 20, 24, 7, 5, 64, 64, "gelu")])        # small grid: the two entries in turn
def test_epilogue_fftconv_bwd(be, B, M, h, w, kh, kw, FH, FW, act):
    res = case_epilogue_fftconv_bwd(be, B=B, M=M, h=h, w=w, kh=kh, kw=kw, FH=FH, FW=FW, act=act)
    _assert_small({k: res[k] for k in ("dx", "dghat_rows", "gz_hat_sum_rows", "pg_rows")},
                  tol=1e-6)
    _assert_small({k: res[k] for k in ("dx_vs_oracle", "gz_vs_oracle")})

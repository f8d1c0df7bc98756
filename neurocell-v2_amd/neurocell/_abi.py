"""ctypes declarations of the C ABI in ``include/neurocell_hip.h``.

``declare(lib)`` attaches argtypes/restypes to a loaded ``ctypes.CDLL`` so every call is
type-checked at the boundary.  ``ENTRY_POINTS`` lists every exported symbol the header
declares; the loader checks all of them on load.
"""
from __future__ import annotations

import ctypes as C

P = C.c_void_p
I = C.c_int
F = C.c_float
SZ = C.c_size_t

NC_OK = 0
NC_ERR_INVALID_ARGUMENT = -1
NC_ERR_UNSUPPORTED = -2
NC_ERR_WORKSPACE = -3
NC_ERR_SCRATCH_LIMIT = -4
NOALLOC_SCRATCH_BYTES = 16 << 20

ACT_IDS = {"identity": 0, "tanh": 1, "sigmoid": 2, "relu": 3, "leaky_relu": 4, "gelu": 5}
CODD_IDS = {"continuous": 0, "annealed": 1, "ste_binary": 2, "ste_ternary": 3}


class ChipDesc(C.Structure):
    """Mirror of ``nc_chip_desc``."""
    _fields_ = [(n, C.c_int32) for n in (
        "H", "W", "kh", "kw", "M", "pad_h", "pad_w", "roi_h", "roi_w", "r0", "r1", "c0", "c1")]


class SpectrumJob(C.Structure):
    """Mirror of ``nc_spectrum_job``."""
    _fields_ = [("x", C.c_void_p), ("xhat", C.c_void_p), ("add", C.c_void_p),
                ("nplanes", C.c_int32), ("hin", C.c_int32), ("win", C.c_int32),
                ("flip", C.c_int32), ("shift_h", C.c_int32), ("shift_w", C.c_int32)]


def spectrum_jobs(*jobs):
    """A ctypes array of SpectrumJob from (x, xhat, add, nplanes, hin, win, flip, sh, sw)
    tuples (pointers as ints or c_void_p / None)."""
    arr = (SpectrumJob * len(jobs))()
    for i, j in enumerate(jobs):
        arr[i] = SpectrumJob(*j)
    return arr


class RowsJob(C.Structure):
    """Mirror of ``nc_rows_job``."""
    _fields_ = [("rows", C.c_void_p), ("out", C.c_void_p), ("len", C.c_int32),
                ("accumulate", C.c_int32), ("nrows", C.c_int32)]


def rows_jobs(*jobs):
    """A ctypes array of RowsJob from (rows, out, len, accumulate, nrows) tuples."""
    arr = (RowsJob * len(jobs))()
    for i, j in enumerate(jobs):
        arr[i] = RowsJob(*j)
    return arr


_SIGS = {
    "nc_version": (I, []),
    "nc_strerror": (C.c_char_p, [I]),
    "nc_codd_fuse_fwd": (I, [P, C.POINTER(ChipDesc), P, P, P, I, F, F, I, I, F, I, P, P, P, P,
                             P, P, P, P, P]),
    "nc_codd_fuse_bwd": (I, [P, C.POINTER(ChipDesc), P, P, P, I, F, F, I, I, F, I, P, P, P, P,
                             P, P, P, P, P, P, P]),
    "nc_step_prologue": (I, [P, C.POINTER(ChipDesc), P, P, P, I, F, F, I, I, F, I, P, P, P, P,
                             P, P, P, I, I, P, I, P, P]),
    "nc_universe_fwd": (I, [P, C.POINTER(ChipDesc), I, I, I, I, F, P, P, P, I, P, P, P]),
    "nc_universe_bwd": (I, [P, C.POINTER(ChipDesc), I, I, I, I, F, P, P, P, I, P, P, P, P, P, P,
                            P]),
    "nc_filter_spectrum_fwd": (I, [P, I, I, I, I, I, P, P]),
    "nc_filter_spectrum_bwd": (I, [P, I, I, I, I, I, I, I, P, P, I, I]),
    "nc_fftconv_fwd": (I, [P, I, I, I, I, I, I, I, I, I, I, P, P, P, P]),
    "nc_fftconv_fwd_ex": (I, [P, I, I, I, I, I, I, I, I, I, I, P, P, P, P, P]),
    "nc_fftconv_fwd_parts": (I, [P, I, I, I, I, I, I, I, I, I, I, P, I, P, P, P, P]),
    "nc_epilogue_fwd_partials": (I, [I, I, I, I]),
    "nc_epilogue_fwd_parts": (I, [P, I, I, I, I, I, F, I, P, P, P, P, P, P, P, P, P, SZ]),
    "nc_plane_spectrum": (I, [P, I, I, I, I, I, I, I, P, P]),
    "nc_plane_spectra": (I, [P, I, I, I, C.POINTER(SpectrumJob)]),
    "nc_spectral_correlate": (I, [P, I, I, I, I, I, I, I, I, P, P, P]),
    "nc_fftconv_spectra": (I, [P, I, I, I, I, I, P, I, P, P]),
    "nc_port_dense_fwd": (I, [P, I, I, I, F, P, P, P]),
    "nc_filter_gate_fwd": (I, [P, I, P, P]),
    "nc_filter_gate_bwd": (I, [P, I, P, P]),
    "nc_filter_patch_bwd": (I, [P, I, I, I, I, I, I, I, P, P, I, I, I, I, I, I, P, P, P, P,
                                SZ]),
    "nc_fftconv_correlate_workspace_size": (SZ, [I, I, I, I, I, I]),
    "nc_fftconv_port_workspace_size": (SZ, [I, I, I, I, I, I, I]),
    "nc_fftconv_port_fwd": (I, [P, I, I, I, I, I, I, I, I, P, P, I, F, I, P, P, P, P, P, P, P,
                                P, P, SZ]),
    "nc_port_dense_bwd": (I, [P, I, I, F, P, P, P]),
    "nc_fftconv_epilogue_partials": (I, [I, I, I, I, I, I]),
    "nc_fftconv_epilogue_fwd": (I, [P, I, I, I, I, I, I, I, I, P, P, I, F, P, P, P, P, P, P, P,
                                    P, SZ]),
    "nc_direct_conv_fwd": (I, [P, I, I, I, I, I, I, I, I, I, I, I, P, I, P, P]),
    "nc_direct_conv_fits": (I, [I, I, I, I, I, I, I, I, I]),
    "nc_direct_conv_dg_partials": (I, [I, I, I, I, I, I]),
    "nc_direct_conv_bwd": (I, [P, I, I, I, I, I, I, I, I, I, I, I, P, P, I, P, I, P, P]),
    "nc_irfft2_pruned_workspace_size": (SZ, [I, I, I]),
    "nc_irfft2_pruned": (I, [P, I, I, I, I, I, I, I, P, P, P, SZ]),
    "nc_spectrum_map": (I, [P, I, I, I, I, I, I, F, F, I, P, P]),
    "nc_standardize_fwd": (I, [P, I, I, P, P, P, P]),
    "nc_standardize_bwd": (I, [P, I, I, P, P, P, P, P]),
    "nc_fftconv_bwd_workspace_size": (SZ, [I, I, I, I]),
    "nc_fftconv_bwd": (I, [P, I, I, I, I, I, I, I, I, I, I, P, P, P, I, P, P, I, I, P, SZ]),
    "nc_fftconv_bwd_ex": (I, [P, I, I, I, I, I, I, I, I, I, I, P, P, P, I, P, P, I, I, P, I, P,
                              SZ]),
    "nc_fftconv_bwd_hat": (I, [P, I, I, I, I, I, I, I, P, P, P, P, P, I, I, P, SZ]),
    "nc_fftconv_bwd_partials": (I, [I, I, I, I]),
    "nc_fftconv_bwd_parts": (I, [P, I, I, I, I, I, I, I, I, I, I, P, P, P, I, P, P, I, I, P, I,
                                 P, SZ]),
    "nc_epilogue_workspace_size": (SZ, [I, I, I, I]),
    "nc_epilogue_fwd": (I, [P, I, I, I, I, I, F, I, P, P, P, P, P, P, P, P, P, SZ]),
    "nc_epilogue_bwd": (I, [P, I, I, I, I, I, F, I, P, P, P, P, P, P, P, P, P, P, P, P, P, I,
                            I, P, SZ]),
    "nc_epilogue_bwd_noalloc": (I, [P, I, I, I, I, I, F, I, P, P, P, P, P, P, P, P, P, P, P,
                                    P, P, I, I]),
    "nc_epilogue_bwd_partials": (I, [I, I, I, I]),
    "nc_epilogue_bwd_parts": (I, [P, I, I, I, I, I, F, I, P, P, P, P, P, P, P, P, P, P, SZ, P,
                                  SZ]),
    "nc_port_bwd_parts": (I, [P, I, I, I, I, I, I, F, I, P, P, P, P, P, P, P, P, P, P, P, SZ, P,
                              SZ]),
    "nc_epilogue_fftconv_bwd_parts": (I, [P, I, I, I, I, I, F, P, P, P, P, P, P, P, P, P, SZ, I,
                                          I, I, I, I, I, P, P, I, P, P, I, I, P, I, P, SZ, P,
                                          SZ]),
    "nc_rows_sum": (I, [P, I, C.POINTER(RowsJob)]),
    "nc_port_fwd": (I, [P, I, I, I, I, I, I, F, I, P, P, P, P, P, P, P, P, P, P, SZ]),
    "nc_port_bwd": (I, [P, I, I, I, I, I, I, F, I, P, P, P, P, P, P, P, P, P, P, P, P, I, P,
                        SZ]),
    "nc_adaptive_stats": (I, [P, C.POINTER(ChipDesc), P, P, P, P, I, I, F, F, F, F, P, P]),
    "nc_inject_roi": (I, [P, I, I, P, I, P, P]),
    "nc_mse_loss": (I, [P, I, P, P, P, P]),
    "nc_packed_accuracy": (I, [P, I, I, P, P, P, P]),
    "nc_adamw_step": (I, [P, I, P, P, P, P, P, P, I, F, F, F, F]),
}

ENTRY_POINTS = tuple(_SIGS)


class NeurocellError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def declare(lib: C.CDLL) -> C.CDLL:
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def check(lib: C.CDLL, status: int, what: str) -> None:
    if status != NC_OK:
        msg = lib.nc_strerror(status)
        raise NeurocellError(f"{what} failed with status {status}: "
                             f"{msg.decode() if msg else '?'}")

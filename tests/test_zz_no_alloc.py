"""The allocation-free epilogue backward (``nc_epilogue_bwd_noalloc``) on the MI355X, through
the C ABI: bit for bit the results of ``nc_epilogue_bwd`` (same kernels, same reduction
order) on consecutive calls that share the file-scope scratch - a config-0-sized call, then
a smaller one (stale scratch contents must not leak into it), then one on the tiled
(N > 8192) pipeline - and a clear error beyond the scratch maximum."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(B, M, h, w, hb, seed):
    rng = np.random.default_rng(seed)
    z = (rng.normal(size=(B, M, h, w)) * 2 + 0.5).astype(np.float32)
    d = rng.normal(size=(M, h, w)).astype(np.float32)
    wv, bv = rng.normal(size=(h, w)).astype(np.float32), rng.normal(size=(h, w)).astype(np.float32)
    sv = rng.uniform(size=(h, w)).astype(np.float32)
    gy = rng.normal(size=(B, h, w)).astype(np.float32)
    return [torch.from_numpy(a).cuda() for a in (z, d, wv, sv, bv, gy)]


def _run(lib, noalloc, B, M, h, w, hb, ins, mean, rstd):
    from neurocell._lib import ptr, stream_ptr
    z, d, wv, sv, bv, gy = ins
    f = dict(device="cuda", dtype=torch.float32)
    outs = [torch.full((B, M, h, w), 3.0, **f), torch.full((M, h, w), 3.0, **f)] + \
        [torch.full((h, w), 3.0, **f) for _ in range(3)]
    gz, gdb, gw, gs, gb = outs
    args = [stream_ptr(), B, M, h, w, 1, 0.0, hb, ptr(z), ptr(d), ptr(wv), ptr(sv), ptr(bv),
            ptr(mean), ptr(rstd), ptr(gy), ptr(gz), ptr(gdb), ptr(gw), ptr(gs), ptr(gb), 0, 0]
    if noalloc:
        rc = lib.nc_epilogue_bwd_noalloc(*args)
    else:
        nb = lib.nc_epilogue_workspace_size(B, M, h, w)
        ws = torch.empty(nb // 4 + 1, **f)
        rc = lib.nc_epilogue_bwd(*args, ptr(ws), ws.numel() * 4)
    assert rc == 0, lib.nc_strerror(rc)
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


@pytest.mark.parametrize("seq", [0])
def test_noalloc_matches_workspace_entry(seq):
    from neurocell._lib import lib as get_lib, ptr, stream_ptr
    lib = get_lib()
    for i, (B, M, h, w, hb) in enumerate([(128, 16, 40, 50, 1),   # config 0's shape
                                          (3, 5, 10, 12, 0),       # smaller, after it
                                          (2, 3, 96, 100, 1)]):    # tiled (N > 8192)
        print(f"[noalloc] call {i}: B={B} M={M} {h}x{w} has_border={hb}", flush=True)
        ins = _case(B, M, h, w, hb, seed=40 + i)
        z, d, wv, sv, bv = ins[:5]
        f = dict(device="cuda", dtype=torch.float32)
        out = torch.empty(B, h, w, **f)
        mean, rstd = torch.empty(B, M, **f), torch.empty(B, M, **f)
        ws = torch.empty(lib.nc_epilogue_workspace_size(B, M, h, w) // 4 + 1, **f)
        rc = lib.nc_epilogue_fwd(stream_ptr(), B, M, h, w, 1, 0.0, hb, ptr(z), ptr(d), ptr(wv),
                                 ptr(sv), ptr(bv), ptr(out), ptr(mean), ptr(rstd), ptr(ws),
                                 ws.numel() * 4)
        assert rc == 0
        ref = _run(lib, False, B, M, h, w, hb, ins, mean, rstd)
        got = _run(lib, True, B, M, h, w, hb, ins, mean, rstd)
        for name, a, b in zip(("gz", "gdb", "gw", "gs", "gb"), got, ref):
            assert np.array_equal(a, b), (i, name)
        assert np.isfinite(got[0]).all()
        if not hb:
            assert (got[1] == 0.0).all()


def test_noalloc_rejects_shapes_beyond_scratch():
    from neurocell import _abi
    from neurocell._lib import lib as get_lib, stream_ptr
    lib = get_lib()
    B, M, h, w = 32, 32, 224, 224  # needs 26.7 MB of scratch
    assert lib.nc_epilogue_workspace_size(B, M, h, w) > _abi.NOALLOC_SCRATCH_BYTES
    rc = lib.nc_epilogue_bwd_noalloc(stream_ptr(), B, M, h, w, 1, 0.0, 1, *([None] * 13), 0, 0)
    assert rc == _abi.NC_ERR_SCRATCH_LIMIT
    assert b"scratch" in lib.nc_strerror(rc)

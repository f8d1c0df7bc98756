"""Shared helpers for the parity tests."""
import numpy as np


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.complex128 if np.iscomplexobj(a) else np.float64)
    b = np.asarray(b, dtype=np.complex128 if np.iscomplexobj(b) else np.float64)
    return float(np.linalg.norm((a - b).ravel()) / (np.linalg.norm(b.ravel()) + 1e-30))


def alu_case(seed, B, out_width=2, depth=4, kernel_size=(23, 13), directions=16):
    """Benchmark-config-0 style inputs: W~N(0,0.1), B~N(0,0.01), S~N(0,1) on (3,62,62),
    filters ~N(0, 1/K) (variance 1/K), 8-bit operand bits + 3-bit opcode as {0,1} cells."""
    from oracle import vnn_oracle as O
    rng = np.random.default_rng(seed)
    geom = O.alu_geometry(kernel_size=kernel_size, directions=directions, depth=depth,
                          out_width=out_width)
    H, W = geom.grid_shape
    kh, kw = kernel_size
    cell = np.stack([rng.normal(0, 0.1, (H, W)), rng.normal(0, 0.01, (H, W)),
                     rng.normal(0, 1.0, (H, W))]).astype(np.float32)
    filt = rng.normal(0, 1.0 / np.sqrt(kh * kw), (directions, 1, kh, kw)).astype(np.float32)
    a = rng.integers(0, 256, size=B, dtype=np.uint8)
    b = rng.integers(0, 256, size=B, dtype=np.uint8)
    op = rng.integers(0, 8, size=B, dtype=np.uint8)
    x = np.zeros((B, 3, 8, 1), np.float32)
    x[:, 0, :, 0] = np.unpackbits(a[:, None], axis=1)
    x[:, 1, :, 0] = np.unpackbits(b[:, None], axis=1)
    x[:, 2, :, 0] = np.unpackbits(op[:, None], axis=1)
    oh, ow = geom.out_size
    y = rng.integers(0, 2, size=(B, oh, ow)).astype(np.float32)
    return geom, cell, filt, x, y


def config_geometry(cfg, depth=None, directions=None):
    """The oracle's restatement of a benchmark config's chip (``neurocell.configs``)."""
    from oracle import vnn_oracle as O
    d = cfg.depth if depth is None else depth
    m = cfg.directions if directions is None else directions
    if cfg.in_port is None:
        return O.alu_geometry(kernel_size=cfg.kernel, directions=m, depth=d, out_width=2)
    (ir, ic), isz = cfg.in_port
    (orr, oc), osz = cfg.out_port
    return O.Geometry(tuple(cfg.grid), tuple(cfg.kernel), m, d,
                      [("rect", (ir, ic), tuple(isz))], ("rect", (orr, oc), tuple(osz)))


def _chunks(B, chunk, threads):
    if chunk is None:  # small chunks keep the oracle's arrays in cache
        chunk = max(1, min(32, -(-B // threads)))
    return [(i, min(B, i + chunk)) for i in range(0, B, chunk)]


def oracle_forward_batched(cell, filt, x, geom, chunk=None, threads=8, states=False, **kw):
    """``oracle.propagate`` over sample chunks on a thread pool (NumPy and scipy.fft release
    the GIL).  Samples are independent in the forward pass (every standardisation is per
    (b, m) plane), so the concatenated outputs equal one call on the whole batch.  With
    ``states`` also returns the step states x_t (t = 0..d-1) as a list of (B, h, w)."""
    from concurrent.futures import ThreadPoolExecutor
    from oracle import vnn_oracle as O
    parts = _chunks(x.shape[0], chunk, threads)
    with ThreadPoolExecutor(threads) as ex:
        res = list(ex.map(lambda p: O.propagate(cell, filt, x[p[0]:p[1]], geom, **kw), parts))
    out = np.concatenate([r[0] for r in res], axis=0)
    if not states:
        return out
    xs = [np.concatenate([r[1]["xs"][t] for r in res], axis=0)
          for t in range(len(res[0][1]["xs"]))]
    return out, xs


def oracle_vjp_batched(cell, filt, x, geom, g_out, chunk=None, threads=8, **kw):
    """``oracle.propagate_vjp`` over sample chunks on a thread pool.  The loss is a sum over
    samples and the parameters are shared, so the parameter gradients of the whole batch are
    the sums of the chunks' gradients (added in float64)."""
    from concurrent.futures import ThreadPoolExecutor
    from oracle import vnn_oracle as O
    parts = _chunks(x.shape[0], chunk, threads)
    with ThreadPoolExecutor(threads) as ex:
        res = list(ex.map(lambda p: O.propagate_vjp(cell, filt, x[p[0]:p[1]], geom,
                                                    g_out[p[0]:p[1]], **kw), parts))
    out = np.concatenate([r[0] for r in res], axis=0)
    gc = np.sum([np.asarray(r[1], np.float64) for r in res], axis=0)
    gf = np.sum([np.asarray(r[2], np.float64) for r in res], axis=0)
    return out, gc, gf

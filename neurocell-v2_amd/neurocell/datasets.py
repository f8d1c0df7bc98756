"""ALU arithmetic / logic datasets staged in device memory (datasets.py:1-179).

The generators draw from NumPy's global random state in the reference's order - operands,
then (for the ALU) control codes, then the uniform noise of each bit plane - so a seeded run
yields the reference's data; labels come from the 8-bit ALU truth table in uint8 arithmetic
(wrapping).  ``prepare_alu_device_dataset`` makes the reference's 80/20 split
(``sklearn.model_selection.train_test_split``, ``random_state=split_seed``) over whole
batches and stages contiguous float32 / uint8 tensors on the device once, in the layouts the
trainer's epochs take: x (nb, B, 3, n, 1), y (nb, B, n), y_packed (nb, B, 1).
"""
from __future__ import annotations

from typing import NamedTuple

import numpy as np
import torch


class ALUDeviceDataset(NamedTuple):
    """Device-resident ALU dataset (datasets.py:19-37).  For samples=128000, batch_size=128,
    test_size=0.2, n=8: x_train (800,128,3,8,1) f32, y_train (800,128,8) f32, y_train_packed
    (800,128,1) u8, and the (200, ...) test counterparts."""
    x_train: torch.Tensor
    y_train: torch.Tensor
    y_train_packed: torch.Tensor
    x_test: torch.Tensor
    y_test: torch.Tensor
    y_test_packed: torch.Tensor


def _bits(values_u8: np.ndarray, n: int) -> np.ndarray:
    # most significant bit first along the last axis (values have a trailing axis of 1)
    return np.unpackbits(values_u8, axis=2, count=n)


def _noisy(bits: np.ndarray, noise: np.ndarray) -> np.ndarray:
    return bits.astype(np.float32) + noise


def generate_arithmetic(samples: int, operation: str = "add", n: int = 8,
                        batch_size: int = 64, noise_level: float = 0.2):
    """datasets.py:40-74: operands uniform in [1, 2^(n-1)), result of ``add`` / ``minus`` /
    ``xor`` in uint8 arithmetic; returns (X1f, X2f, Y_raw), X* (nb, B, n) bits plus uniform
    noise in [-noise_level, noise_level), Y_raw (nb, B, n) uint8 bits."""
    hi = 2 ** (n - 1)
    nb = samples // batch_size
    shape = (nb, batch_size, 1)
    a = np.random.randint(1, hi, size=shape, dtype=np.uint8)
    b = np.random.randint(1, hi, size=shape, dtype=np.uint8)
    op = operation.lower()
    if op == "minus":
        res = a - b
    elif op == "xor":
        res = a ^ b
    else:
        res = a + b
    xa, xb, y = _bits(a, n), _bits(b, n), _bits(res, n)
    na = np.random.uniform(-noise_level, noise_level, size=xa.shape)
    nbits = np.random.uniform(-noise_level, noise_level, size=xb.shape)
    return _noisy(xa, na), _noisy(xb, nbits), y


def alu_truth_table(a: np.ndarray, b: np.ndarray, ctrl: np.ndarray) -> np.ndarray:
    """The ALU's uint8 result for operands a, b and control code ctrl (datasets.py:95-115):
    0/4 -> a, 1 -> a+1, 2/8 -> a+b, 3 -> a+b+1, 5 -> a-1, 6 -> a-b, 7 -> a-b-1, any other
    code -> a; sums and differences wrap modulo 256."""
    a16, b16, c = a.astype(np.int32), b.astype(np.int32), ctrl.astype(np.int32)
    out = a16.copy()
    table = ((1, a16 + 1), (2, a16 + b16), (8, a16 + b16), (3, a16 + b16 + 1), (5, a16 - 1),
             (6, a16 - b16), (7, a16 - b16 - 1))
    for code, val in table:
        out = np.where(c == code, val, out)
    return (out % 256).astype(np.uint8)


def generate_arithmetic_logic(samples: int, n: int = 8, ctrl_bits: int = 4,
                              batch_size: int = 64, noise_level: float = 0.2):
    """datasets.py:77-130: operands in [1, 2^(n-1)), control codes in [1, 2^ctrl_bits);
    returns (X1f, X2f, Cf, Y_raw) as ``generate_arithmetic`` plus the noisy control bits."""
    hi = 2 ** (n - 1)
    nb = samples // batch_size
    shape = (nb, batch_size, 1)
    a = np.random.randint(1, hi, size=shape, dtype=np.uint8)
    b = np.random.randint(1, hi, size=shape, dtype=np.uint8)
    c = np.random.randint(1, 2 ** ctrl_bits, size=shape, dtype=np.uint8)
    y = _bits(alu_truth_table(a, b, c), n)
    xa, xb, xc = _bits(a, n), _bits(b, n), _bits(c, n)
    na = np.random.uniform(-noise_level, noise_level, size=xa.shape)
    nbits = np.random.uniform(-noise_level, noise_level, size=xb.shape)
    nc = np.random.uniform(-noise_level, noise_level, size=xc.shape)
    return _noisy(xa, na), _noisy(xb, nbits), _noisy(xc, nc), y


def prepare_alu_device_dataset(samples: int = 128000, n: int = 8, ctrl_bits: int = 4,
                               batch_size: int = 128, noise_level: float = 0.2,
                               test_size: float = 0.2, split_seed: int = 42,
                               device=None) -> ALUDeviceDataset:
    """datasets.py:133-179: the ALU dataset split 80/20 over batches and staged on ``device``
    (default: the current GPU) once."""
    from sklearn.model_selection import train_test_split

    x1, x2, xc, y = generate_arithmetic_logic(samples=samples, n=n, ctrl_bits=ctrl_bits,
                                              batch_size=batch_size, noise_level=noise_level)
    x = np.concatenate([x1, x2, xc], axis=-1)  # (nb, B, 3n)
    x_tr, x_te, y_tr, y_te = train_test_split(x, y, test_size=test_size,
                                              random_state=split_seed)

    def ports(a):  # (nb, B, 3n) -> (nb, B, 3, n, 1) float32
        return np.ascontiguousarray(
            np.stack(np.split(a, 3, axis=2), axis=2).astype(np.float32)[..., None])

    dev = torch.device("cuda") if device is None else torch.device(device)

    def put(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    return ALUDeviceDataset(
        x_train=put(ports(x_tr)), y_train=put(y_tr.astype(np.float32)),
        y_train_packed=put(np.packbits(y_tr, axis=2)),
        x_test=put(ports(x_te)), y_test=put(y_te.astype(np.float32)),
        y_test_packed=put(np.packbits(y_te, axis=2)))

"""ALU dataset generators (datasets.py:40-179) on the CPU: the truth table against worked
values, and every generated sample against its own operands - the operands and control code
are decoded from the noisy bits, so labels, bit order, noise range, packing and the batch
split are each checked against data the generator did not compute them from.  Whether a seeded
run reproduces the reference's exact random stream is not checked here (the reference cannot
be run in this image); the draws follow its order."""
import numpy as np
import pytest

from neurocell.datasets import (alu_truth_table, generate_arithmetic, generate_arithmetic_logic,
                                prepare_alu_device_dataset)

WEIGHTS = np.array([128, 64, 32, 16, 8, 4, 2, 1])


def _decode(xf, delta):
    bits = np.round(xf).astype(np.int64)
    assert set(np.unique(bits)) <= {0, 1}
    assert np.all(np.abs(xf - bits) <= delta)
    return (bits * WEIGHTS[-bits.shape[-1]:]).sum(-1)


@pytest.mark.parametrize("a,b,expect", [
    (5, 3, {0: 5, 1: 6, 2: 8, 3: 9, 4: 5, 5: 4, 6: 2, 7: 1, 8: 8, 9: 5, 15: 5}),
    (1, 127, {5: 0, 6: 130, 7: 129, 2: 128, 3: 129}),       # differences wrap modulo 256
    (127, 127, {3: 255, 1: 128, 6: 0, 7: 255, 8: 254}),
])
def test_truth_table_worked_values(a, b, expect):
    for c, want in expect.items():
        got = alu_truth_table(np.uint8([a]), np.uint8([b]), np.uint8([c]))[0]
        assert int(got) == want, (a, b, c, int(got), want)


def test_alu_generator_labels_and_noise():
    np.random.seed(3)
    x1, x2, xc, y = generate_arithmetic_logic(samples=640, batch_size=64, noise_level=0.2)
    assert x1.shape == x2.shape == xc.shape == y.shape == (10, 64, 8)
    assert y.dtype == np.uint8 and set(np.unique(y)) <= {0, 1}
    a, b, c = _decode(x1, 0.2), _decode(x2, 0.2), _decode(xc, 0.2)
    assert a.min() >= 1 and a.max() <= 127 and b.min() >= 1 and b.max() <= 127
    assert c.min() >= 1 and c.max() <= 15
    assert len(np.unique(c)) == 15  # every code 1..15 drawn at this size
    res = (y.astype(np.int64) * WEIGHTS).sum(-1)
    want = alu_truth_table(a.astype(np.uint8), b.astype(np.uint8), c.astype(np.uint8))
    assert np.array_equal(res, want.astype(np.int64))
    # the noise is a continuous uniform draw on each bit, not a copy across planes
    assert np.abs(x1 - np.round(x1)).std() > 0.05
    assert not np.allclose(x1 - np.round(x1), x2 - np.round(x2))
    # the same seed gives the same data
    np.random.seed(3)
    again = generate_arithmetic_logic(samples=640, batch_size=64, noise_level=0.2)
    assert all(np.array_equal(p, q) for p, q in zip((x1, x2, xc, y), again))


@pytest.mark.parametrize("op,fn", [("add", lambda a, b: a + b), ("minus", lambda a, b: a - b),
                                   ("xor", lambda a, b: a ^ b)])
def test_arithmetic_generator(op, fn):
    np.random.seed(11)
    x1, x2, y = generate_arithmetic(samples=256, operation=op, batch_size=32, noise_level=0.1)
    assert x1.shape == y.shape == (8, 32, 8)
    a, b = _decode(x1, 0.1), _decode(x2, 0.1)
    res = (y.astype(np.int64) * WEIGHTS).sum(-1)
    assert np.array_equal(res, fn(a, b) % 256)


def test_prepare_split_layout_and_packing():
    np.random.seed(5)
    ds = prepare_alu_device_dataset(samples=1280, batch_size=64, device="cpu")
    assert tuple(ds.x_train.shape) == (16, 64, 3, 8, 1)
    assert tuple(ds.x_test.shape) == (4, 64, 3, 8, 1)
    assert tuple(ds.y_train.shape) == (16, 64, 8) and tuple(ds.y_test.shape) == (4, 64, 8)
    assert tuple(ds.y_train_packed.shape) == (16, 64, 1)
    assert str(ds.x_train.dtype) == str(ds.y_train.dtype) == "torch.float32"
    assert str(ds.y_train_packed.dtype) == "torch.uint8"
    for x, yf, yp in ((ds.x_train, ds.y_train, ds.y_train_packed),
                      (ds.x_test, ds.y_test, ds.y_test_packed)):
        x, yf, yp = x.numpy()[..., 0], yf.numpy(), yp.numpy()[..., 0]
        a, b, c = (_decode(x[:, :, k], 0.2) for k in range(3))  # port rows: A, B, control
        res = (yf.astype(np.int64) * WEIGHTS).sum(-1)
        assert np.array_equal(res, yp.astype(np.int64))
        want = alu_truth_table(a.astype(np.uint8), b.astype(np.uint8), c.astype(np.uint8))
        assert np.array_equal(res, want.astype(np.int64))
    # the split partitions the generated batches: regenerate and match each batch once
    np.random.seed(5)
    x1, x2, xc, y = generate_arithmetic_logic(samples=1280, batch_size=64)
    full = np.stack([x1, x2, xc], axis=2).astype(np.float32)
    got = np.concatenate([ds.x_train.numpy()[..., 0], ds.x_test.numpy()[..., 0]])
    idx = [int(np.flatnonzero((full == g).all(axis=(1, 2, 3)))[0]) for g in got]
    assert sorted(idx) == list(range(20))

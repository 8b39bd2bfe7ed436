"""Pins the scan oracle (CPU only): closed forms, brute force, the torch CPU
reference path (bit-equal), float64 autograd, the C restatement, and
planted mistakes that must fail."""

import numpy as np
import pytest
import torch

from oracle import native
from oracle import scan as osc


def _u(shape, seed):
    return np.random.default_rng(seed).uniform(-1, 1, shape).astype(np.float32)


def test_known_values_and_closed_forms():
    assert np.array_equal(osc.cumsum_f32([[1, 2, 3]]), np.array([[1, 3, 6]], np.float32))
    d = 5000
    assert np.array_equal(osc.cumsum_f32(np.ones((2, d))), np.tile(np.arange(1, d + 1), (2, 1)))
    a = np.arange(d, dtype=np.float32)[None]
    assert np.array_equal(osc.cumsum_f32(a)[0], (np.arange(d) * (np.arange(d) + 1) // 2))
    c = np.full((3, 777), -1000, np.int32)
    assert np.array_equal(osc.cumsum_i64(c), -1000 * np.tile(np.arange(1, 778), (3, 1)))
    assert np.array_equal(osc.reverse_cumsum_f32(np.ones((1, 4))), [[4, 3, 2, 1]])


def test_brute_force_small():
    x = _u((3, 57), 1)
    assert np.array_equal(osc.cumsum_f32(x), osc.cumsum_loops(x).astype(np.float32))
    xi = np.random.default_rng(2).integers(-1000, 1001, (4, 91)).astype(np.int32)
    assert np.array_equal(osc.cumsum_i64(xi), osc.cumsum_loops(xi))


@pytest.mark.parametrize("shape", [(4, 65536), (16, 4096), (3, 100003)])
def test_matches_torch_cpu_cumsum_bitwise(shape):
    x = _u(shape, shape[1])
    t = torch.cumsum(torch.from_numpy(x), dim=-1).numpy()
    assert np.array_equal(osc.cumsum_f32(x), t)
    xn = np.random.default_rng(7).standard_normal(shape).astype(np.float32)
    assert np.array_equal(osc.cumsum_f32(xn), torch.cumsum(torch.from_numpy(xn), -1).numpy())


def test_int_matches_torch_cpu_exactly():
    xi = np.random.default_rng(3).integers(-1000, 1001, (8, 65536)).astype(np.int32)
    t = torch.cumsum(torch.from_numpy(xi), dim=-1)
    assert t.dtype == torch.int64
    assert np.array_equal(osc.cumsum_i64(xi), t.numpy())


def test_backward_matches_autograd_and_flip_identity():
    g = np.random.default_rng(4).standard_normal((5, 3000)).astype(np.float32)
    x = torch.zeros(5, 3000, dtype=torch.float64, requires_grad=True)
    torch.cumsum(x, -1).backward(torch.from_numpy(g).double())
    ref = x.grad.numpy().astype(np.float32)
    assert np.array_equal(osc.reverse_cumsum_f32(g), ref)
    assert np.array_equal(osc.reverse_cumsum_f32(g),
                          np.flip(osc.cumsum_f32(np.flip(g, -1)), -1))
    tg = osc.torch_cpu_backward(torch.zeros(5, 3000), torch.from_numpy(g)).numpy()
    assert np.allclose(osc.reverse_cumsum_f32(g), tg, atol=1e-4, rtol=1e-5)


def test_wrap_variant():
    x = np.array([[2**31 - 1, 1, 2**31 - 1, -(2**31), -5]], np.int32)
    exact = [2**31 - 1, 2**31, 2**32 - 1, 2**31 - 1, 2**31 - 6]
    want = [(v + 2**31) % 2**32 - 2**31 for v in exact]
    assert np.array_equal(osc.cumsum_i64(x)[0], exact)
    assert np.array_equal(osc.cumsum_i32_wrap(x)[0], want)


def test_c_restatement_agrees():
    L = native.lib()
    if L is None:
        pytest.skip("oracle/lib/liboracle.so not built")
    x = _u((6, 9000), 5)
    assert np.array_equal(native.scan_f32(x), osc.cumsum_f32(x))
    assert np.array_equal(native.scan_f32(x, reverse=True), osc.reverse_cumsum_f32(x))
    xi = np.random.default_rng(6).integers(-1000, 1001, (6, 9000)).astype(np.int32)
    assert np.array_equal(native.scan_i32(xi), osc.cumsum_i64(xi))


def _exclusive(x):
    y = osc.cumsum_f32(x)
    return np.concatenate([np.zeros_like(y[:, :1]), y[:, :-1]], axis=1)


def _f32_accumulation(x):
    return np.cumsum(np.asarray(x, np.float32), axis=-1, dtype=np.float32)


def _reverse_off_by_one(g):
    r = osc.reverse_cumsum_f32(g)
    return np.concatenate([r[:, 1:], np.zeros_like(r[:, :1])], axis=1)


@pytest.mark.parametrize("bad", [_exclusive, _f32_accumulation, _reverse_off_by_one])
def test_planted_mistakes_are_caught(bad):
    x = _u((4, 65536), 11)
    t = torch.cumsum(torch.from_numpy(x), -1).numpy()
    if bad is _reverse_off_by_one:
        assert not np.array_equal(bad(x), osc.reverse_cumsum_f32(x))
    else:
        assert not np.array_equal(bad(x), t)

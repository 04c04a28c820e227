"""Shared helpers of the GPU parity tests: seeded host inputs (numpy, so the oracle and the GPU
consume identical bytes), upload, and the reference's elementwise tolerance rule
|got - ref| <= atol + rtol |ref| (reference tests/test_kernels.py:20-26)."""
import numpy as np
import pytest


def rng(seed):
    return np.random.default_rng(seed)


def h16(r, *shape, sd=1.0):
    return (r.standard_normal(shape) * sd).astype(np.float16)


def cuda(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def check(name, got, ref, atol, rtol=0.0):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"{name}: shape {got.shape} vs {ref.shape}"
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not np.isnan(got).any(), f"{name}: NaN in output"
    assert not bad.any(), f"{name}: {int(bad.sum())} of {bad.size} outside tolerance, max_abs_err={err.max():.3e}"


def bits(a):
    return np.asarray(a).view(np.uint16)


def interleave(g, u):
    I, H = g.shape
    return np.stack([g.reshape(I // 16, 16, H), u.reshape(I // 16, 16, H)], 1).reshape(2 * I, H)


gpu = pytest.mark.gpu

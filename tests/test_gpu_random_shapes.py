"""Seeded random shapes through the automatic path choice.

Each case draws m (weighted to the thresholds between paths: 1, 2-8, 8-9,
16, 31-33, 63-65 and above), a group, the four transpose layouts, n a
multiple of 8 g or not, k a multiple of the group, of 16 or neither, and 1-3
batched instances (hundreds for the instance kernels), in five kinds that aim
at each path (80 cases: 11 one-hot MFMA, 15 gemv-rows, 6 gemv-row-pairs, 14
gemv-direct, 17 gram-mfma, 16 general, one gemv-pairs). Whatever path the
shape takes (general, gemv-direct, gemv-pairs, gemv-rows, gemv-row-pairs,
onehot-mfma with or without k split, gram-mfma), every output must be within
1e-5 of the float64 product of the decoded operands, row by row against that
row's largest output (the first, middle and last instance of a batch), and
the status word must stay clear.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import image, run_plan, say

pytestmark = pytest.mark.gpu

TOL = 1e-5
ROWS = [1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 31, 32, 33, 63, 64, 65, 100, 130, 200]


def _small(rng):
    """Any layout, sizes where the general kernel or gemv-direct serves."""
    group = int(rng.choice([8, 16, 32]))
    flags = int(rng.choice([0, 0, 1, 2, 3]))
    m = int(rng.choice(ROWS))
    n = 8 * group * int(rng.integers(1, 9)) if rng.random() < 0.8 else int(rng.integers(8, 1500))
    kind = rng.random()
    if kind < 0.5:
        k = group * int(rng.integers(1, 3000 // group))
    elif kind < 0.8:
        k = 16 * int(rng.integers(1, 200))
    else:
        k = int(rng.integers(5, 3000))
    count = int(rng.choice([1, 1, 2, 3]))
    while m * n * k * count > 1 << 24:
        k = max(group, k // 2)
        if m * n * k * count > 1 << 24:
            n = max(8 * group, n // 2)
    return m, n, k, group, flags, count


def _large(rng):
    """One product over at least 2^20 weights: one-hot MFMA (with k split on
    small grids), the chunked row GEMV, gemv-pairs."""
    group = int(rng.choice([8, 16, 32]))
    flags = int(rng.choice([0, 0, 0, 1]))
    m = int(rng.choice(ROWS))
    n = 8 * group * int(rng.integers(2, 20))
    unit = int(rng.choice([group, 16]))
    kmin = -(-(1 << 20) // (n * unit))
    k = unit * int(rng.integers(kmin, kmin + max(2, (1 << 22) // (n * unit) - kmin)))
    while m * n * k > 1 << 27 and n * k > 1 << 21:
        k = max(unit, k // 2 // unit * unit)
    return m, n, k, group, flags, 1


def _batched(rng):
    """Batches of 1-8 rows that fill the chip with instances: gemv-pairs and
    gemv-row-pairs."""
    group = int(rng.choice([8, 16, 32]))
    m = int(rng.choice([1, 2, 3, 4, 5, 8]))
    n = 8 * group * int(rng.choice([4, 8, 16]))
    k = 8 * group * int(rng.integers(2, 12))
    while n * k > 1 << 20 and k > 16 * group:
        k -= 8 * group
    count = -(-(1 << 25) // (n * k)) + int(rng.integers(0, 8))
    return m, n, k, group, 0, count


def _gram(rng):
    """B stored (n, k), both operands grouped along k: gram-mfma."""
    group = int(rng.choice([8, 16, 32]))
    m = int(rng.choice([16, 64, 100, 130, 200]))
    n = int(rng.integers(64, 1500))
    k = group * int(rng.integers(8, 4096 // group))
    while m * n * k < 1 << 22:
        n *= 2
    return m, n, k, group, 2, 1


def _case(i):
    rng = np.random.default_rng(1000 + i)
    kind = (_small, _large, _large, _batched, _gram)[i % 5]
    return kind(rng)


CASES = [_case(i) for i in range(80)]


def _decoded(codes, book, count, shape, group):
    from oracle import vq4_numpy as o
    return o.decode(codes, book, count, group).reshape(shape).astype(np.float64)


@pytest.mark.parametrize("case", range(len(CASES)))
def test_random_shape_within_tolerance(vqdev, case):
    m, n, k, group, flags, count = CASES[case]
    rng = np.random.default_rng(7 * case + 1)
    items = []
    for _ in range(count):
        a_codes, a_book = image(rng, m * k, group, 1.0)
        b_codes, b_book = image(rng, k * n, group, 0.02)
        items.append((a_codes, a_book, b_codes, b_book))
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in items]) for s in range(4))
    words = (2, m, n, k, group, 16, flags, 0)
    path = vqdev.path_name(words, count=count)
    say("random shape", case, m, n, k, group, flags, count, path)
    out, status = run_plan(vqdev, words, ops, 4 * m * n * count, np.float32, count=count)
    assert status == 0
    out = out.reshape(count, m, n)
    for i in sorted({0, count // 2, count - 1}):
        a_codes, a_book, b_codes, b_book = items[i]
        a = _decoded(a_codes, a_book, m * k, (k, m) if flags & 1 else (m, k), group)
        b = _decoded(b_codes, b_book, k * n, (n, k) if flags & 2 else (k, n), group)
        ref = (a.T if flags & 1 else a) @ (b.T if flags & 2 else b)
        scale = np.abs(ref).max(axis=1, keepdims=True)
        err = np.abs(out[i] - ref) / np.maximum(scale, np.finfo(np.float64).tiny)
        assert err.max() <= TOL, f"instance {i} on {path}: row-relative error {err.max():.3g}"


@pytest.mark.parametrize("case", range(len(CASES)))
def test_random_shape_dense_activations(vqdev, case):
    """The same shapes (one instance) with dense FP32 activations
    (ack_vq_matmul_dense: onehot-mfma, its bf16 planes, gemv-direct,
    gemv-pairs, gemv-rows, gram is not offered, general), rows of very
    different magnitude: every row within 1e-5 of the float64 product."""
    m, n, k, group, flags, _ = CASES[case]
    rng = np.random.default_rng(11 * case + 5)
    b_codes, b_book = image(rng, k * n, group, 0.02)
    x = rng.standard_normal((k, m) if flags & 1 else (m, k)).astype(np.float32)
    if m > 2:
        x.reshape(-1)[::7] *= np.float32(1e3)
    words = (2, m, n, k, group, 16, flags, 0)
    path = vqdev.dense_path_name(words)
    say("random shape dense", case, m, n, k, group, flags, path)
    device = vqdev.device
    bufs = [device.buffer(a.nbytes) for a in (x, b_codes, b_book)]
    out, status = device.buffer(4 * m * n), device.buffer(4)
    try:
        for b_, a in zip(bufs, (x, b_codes, b_book)):
            b_.upload(a)
        status.upload(np.zeros(1, np.uint32))
        vqdev.run_dense(words, *bufs, out, status)
        assert int(status.download(np.uint32)[0]) == 0
        y = out.download(np.float32).reshape(m, n)
    finally:
        for b_ in bufs + [out, status]:
            b_.free()
    a = x.astype(np.float64)
    b = _decoded(b_codes, b_book, k * n, (n, k) if flags & 2 else (k, n), group)
    ref = (a.T if flags & 1 else a) @ (b.T if flags & 2 else b)
    scale = np.abs(ref).max(axis=1, keepdims=True)
    err = np.abs(y - ref) / np.maximum(scale, np.finfo(np.float64).tiny)
    assert err.max() <= TOL, f"{path}: row-relative error {err.max():.3g}"

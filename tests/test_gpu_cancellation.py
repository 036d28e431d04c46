"""Cancellation-heavy activations on the reordered GEMV paths.

Activations come in pairs x, -x(1 + eps) on rows of B that carry the same
codes, so every output is eps times smaller than the sum of magnitudes that
flows through it. K = 4096 and 14336, eps from 1e-1 to 1e-3. No FP32 order
holds 1e-5 of max|y| here: the reference's sequential loop
(vq4.comp:168-174) rounds each partial sum to the size of one product, an
error about u / eps relative to the output (measured 3e-6 to 1e-4 for these
cases), and any other order does the same.

What each path guarantees, and what is checked output by output against the
float64 product of the decoded operands:

* the fixed-point GEMVs (gemv-pairs, gemv-row-pairs, gemv-rows) round each
  activation once to a window scale 2^-s with 2^s M (1 + 2^-8) < 2^31, M the
  window's larger signed mass max(P, N); so for output t
      |y' - y| <= max_e |C_B[e][t]| (K 2^-31 (1 + 2^-8)(1 + 2^-11) M
                                     + (K / 256 + 17) u L1),
  the second term the FP32 roundings (window and split sums, the 16-term
  product), M and L1 over the whole row (a window's are smaller);
* gemv-direct (FP32 multiply-adds in another order) is held to the bound of
  any FP32 summation order, gamma_K sum_k |x_k w_kt| -- the class of the
  shader's own rounding error;
* onehot-mfma (from 8 packed or 9 dense rows over large weights) adds each
  activation as three exact bf16 terms in FP32 and then applies the book:
  gamma_(3K + 17) (1 + 2^-7) sum_k |x_k w_kt|.

The shader's own error (the oracle) is reported beside them: on these inputs
the fixed-point paths' errors stay within a few times the shader's, and the
bound, not 1e-5, is what any of these paths guarantees here.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def _weight(rng, k, n, group, pair_rows):
    """Random codes and an N(0, 0.02^2) book; rows 2i + 1 of B copy row 2i's
    codes (pair_rows 1), or the rows of group 2i + 1 copy those of group 2i
    (pair_rows = group: packed activations pair whole groups)."""
    words_per_row = n // (8 * group)
    codes = rng.integers(0, 2 ** 32, (k, words_per_row), dtype=np.uint64).astype(np.uint32)
    blocks = codes.reshape(k // (2 * pair_rows), 2, pair_rows, words_per_row)
    blocks[:, 1] = blocks[:, 0]
    book = (rng.standard_normal((16, group)) * 0.02).astype(np.float32)
    return codes.reshape(-1), book


def _decode(codes, book, k, n, group):
    from oracle import vq4_numpy as o
    return o.decode(codes, book, k * n, group).reshape(k, n).astype(np.float64)


def _fixed_point_bound(x64, book, k, n, group):
    cmax = np.tile(np.abs(book.astype(np.float64)).max(axis=0), n // group)
    p = np.clip(x64, 0, None).sum(axis=1)
    q = np.clip(-x64, 0, None).sum(axis=1)
    quant = k * 2.0 ** -31 * (1 + 2.0 ** -8) * (1 + 2.0 ** -11) * np.maximum(p, q)
    fp32 = (k / 256 + 17) * U * (p + q)
    return (quant + fp32)[:, None] * cmax[None, :]


def _fp32_bound(x64, w64, k):
    return k * U / (1 - k * U) * (np.abs(x64) @ np.abs(w64))


def _report(name, y, y64, oracle_y, bound):
    scale = np.abs(y64).max()
    err = np.abs(y - y64)
    say(name, f"max|y| {scale:.3g}", f"err/max|y| {err.max() / scale:.2e}",
        f"bound/max|y| {bound.max() / scale:.2e}",
        f"shader err/max|y| {np.abs(oracle_y - y64).max() / scale:.2e}"
        if oracle_y is not None else "")
    assert np.all(err <= bound), f"{name}: an output exceeds its bound"


def _dense_pairs(rng, m, k, eps):
    a = rng.standard_normal((m, k // 2)).astype(np.float32)
    x = np.empty((m, k), np.float32)
    x[:, 0::2] = a
    x[:, 1::2] = (-a.astype(np.float64) * (1 + eps)).astype(np.float32)
    return x


def _run_dense(vqdev, words, x, codes, book):
    device = vqdev.device
    bufs = [device.buffer(arr.nbytes) for arr in (x, codes, book)]
    out, status = device.buffer(4 * words[1] * words[2]), device.buffer(4)
    try:
        for b, arr in zip(bufs, (x, codes, book)):
            b.upload(arr)
        status.upload(np.zeros(1, np.uint32))
        vqdev.run_dense(words, *bufs, out, status)
        assert int(status.download(np.uint32)[0]) == 0
        return out.download(np.float32).reshape(words[1], words[2])
    finally:
        for b in bufs + [out, status]:
            b.free()


CASES = [(k, eps) for k in (4096, 14336) for eps in (1e-1, 1e-2, 1e-3)]


@pytest.mark.parametrize("k,eps", CASES)
def test_gemv_pairs_and_direct_under_cancellation(vqdev, oracle, k, eps):
    """One dense activation row: gemv-pairs (test policy) within its
    fixed-point bound, gemv-direct (the automatic choice) within the FP32
    bound."""
    rng = np.random.default_rng(k + int(1 / eps))
    n, group = 2048, 16
    codes, book = _weight(rng, k, n, group, 1)
    w64 = _decode(codes, book, k, n, group)
    x = _dense_pairs(rng, 1, k, eps)
    x64 = x.astype(np.float64)
    y64 = x64 @ w64
    ref, st = oracle.matmul_dense(x, codes, book, 1, n, k, group, 0)
    assert st == 0
    words = (2, 1, n, k, group, 16, 0, 0)
    assert vqdev.dense_path_name(words) == "gemv-direct"
    say("cancellation gemv-direct", k, eps)
    y = _run_dense(vqdev, words, x, codes, book)
    _report("gemv-direct", y, y64, ref, _fp32_bound(x64, w64, k))
    vqdev.device.set_policy(2)
    try:
        say("cancellation gemv-pairs (test policy)", k, eps)
        y = _run_dense(vqdev, words, x, codes, book)
    finally:
        vqdev.device.set_policy(0)
    _report("gemv-pairs", y, y64, ref, _fixed_point_bound(x64, book, k, n, group))


@pytest.mark.parametrize("k,eps", CASES)
def test_gemv_rows_under_cancellation(vqdev, oracle, k, eps):
    """Four dense activation rows stored k x m (flags bit 0), so the row-pair
    bins (gemv-rows) take them under the test policy; each row pairs its own
    values."""
    rng = np.random.default_rng(7 * k + int(1 / eps))
    m, n, group = 4, 2048, 16
    codes, book = _weight(rng, k, n, group, 1)
    w64 = _decode(codes, book, k, n, group)
    x = _dense_pairs(rng, m, k, eps)
    x[1] *= 1e-3                                   # rows of different magnitude
    xt = np.ascontiguousarray(x.T)                 # stored k x m
    x64 = x.astype(np.float64)
    y64 = x64 @ w64
    ref, st = oracle.matmul_dense(xt, codes, book, m, n, k, group, 1)
    assert st == 0
    words = (2, m, n, k, group, 16, 1, 0)
    vqdev.device.set_policy(2)
    try:
        say("cancellation gemv-rows (test policy)", k, eps)
        y = _run_dense(vqdev, words, xt, codes, book)
    finally:
        vqdev.device.set_policy(0)
    _report("gemv-rows", y, y64, ref, _fixed_point_bound(x64, book, k, n, group))


@pytest.mark.parametrize("k,eps", CASES)
def test_gemv_row_pairs_under_cancellation(vqdev, oracle, k, eps):
    """Packed activations (4 rows each) over a batch of 64 weights, the
    automatic gemv-row-pairs choice: the A book holds pairs of entries v,
    -v(1 + eps), groups 2i and 2i + 1 of a row take a pair, and B's rows of
    group 2i + 1 copy those of group 2i."""
    from gpu_util import run_plan
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(11 * k + int(1 / eps))
    m, n, group, count = 4, 2048, 16, 64
    codes, book = _weight(rng, k, n, group, group)
    w64 = _decode(codes, book, k, n, group)
    v = rng.standard_normal((8, group))
    a_book = np.empty((16, group), np.float32)
    a_book[0::2] = v
    a_book[1::2] = -v * (1 + eps)
    groups = m * k // group
    a_codes, xs = [], []
    for _ in range(count):
        pick = rng.integers(0, 8, groups // 2)
        idx = np.empty(groups, np.uint32)
        idx[0::2] = 2 * pick
        idx[1::2] = 2 * pick + 1
        words = np.zeros(groups // 8, np.uint32)
        for lane in range(8):
            words |= idx[lane::8] << np.uint32(4 * lane)
        a_codes.append(words)
        xs.append(o.decode(words, a_book, m * k, group).reshape(m, k).astype(np.float64))
    plan = (2, m, n, k, group, 16, 0, 0)
    assert vqdev.path_name(plan, count=count) == "gemv-row-pairs"
    arrays = (np.concatenate(a_codes), np.tile(a_book.reshape(-1), count),
              np.tile(codes, count), np.tile(book.reshape(-1), count))
    say("cancellation gemv-row-pairs", k, eps, count)
    out, status = run_plan(vqdev, plan, arrays, 4 * m * n * count, np.float32, count=count)
    assert status == 0
    out = out.reshape(count, m, n)
    ref, st = oracle.matmul(a_codes[0], a_book, codes, book, m, n, k, group, 0)
    assert st == 0
    for i in range(count):
        y64 = xs[i] @ w64
        bound = _fixed_point_bound(xs[i], book, k, n, group)
        if i == 0:
            _report("gemv-row-pairs", out[0], y64, ref, bound)
        else:
            assert np.all(np.abs(out[i] - y64) <= bound), f"instance {i}"


def _onehot_bound(x64, w64, k):
    """The one-hot MFMA path's bound: each activation enters as three exact
    bf16 terms (3 k FP32 additions of terms that sum to at most |x| (1 + 2^-7)),
    then the 16-term product with the book: gamma_(3k + 17) sum_k |x_k w_kt|."""
    n_ops = 3 * k + 17
    return n_ops * U / (1 - n_ops * U) * (1 + 2.0 ** -7) * (np.abs(x64) @ np.abs(w64))


@pytest.mark.parametrize("k,eps", CASES)
def test_onehot_mfma_dense_under_cancellation(vqdev, oracle, k, eps):
    """Sixteen dense activation rows on the one-hot MFMA path (k split over
    blocks at this size), the pairs x, -x(1 + eps) of the GEMV cases: every
    output within the bound of its FP32 sums."""
    rng = np.random.default_rng(13 * k + int(1 / eps))
    m, n, group = 16, 2048, 16
    codes, book = _weight(rng, k, n, group, 1)
    w64 = _decode(codes, book, k, n, group)
    x = _dense_pairs(rng, m, k, eps)
    x[1] *= 1e-3
    x64 = x.astype(np.float64)
    ref, st = oracle.matmul_dense(x, codes, book, m, n, k, group, 0)
    assert st == 0
    words = (2, m, n, k, group, 16, 0, 0)
    assert vqdev.dense_path_name(words) == "onehot-mfma"
    say("cancellation onehot-mfma dense", k, eps)
    y = _run_dense(vqdev, words, x, codes, book)
    _report("onehot-mfma dense", y, x64 @ w64, ref, _onehot_bound(x64, w64, k))


@pytest.mark.parametrize("k,eps", CASES)
def test_onehot_mfma_packed_under_cancellation(vqdev, oracle, k, eps):
    """Twelve rows of packed activations on the one-hot MFMA path: the A
    book holds pairs v, -v(1 + eps), groups 2i and 2i + 1 of a row take a
    pair, and B's rows of group 2i + 1 copy those of group 2i."""
    from gpu_util import run_plan
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(17 * k + int(1 / eps))
    m, n, group = 12, 2048, 16
    codes, book = _weight(rng, k, n, group, group)
    w64 = _decode(codes, book, k, n, group)
    v = rng.standard_normal((8, group))
    a_book = np.empty((16, group), np.float32)
    a_book[0::2] = v
    a_book[1::2] = -v * (1 + eps)
    groups = m * k // group
    pick = rng.integers(0, 8, groups // 2)
    idx = np.empty(groups, np.uint32)
    idx[0::2] = 2 * pick
    idx[1::2] = 2 * pick + 1
    a_codes = np.zeros(groups // 8, np.uint32)
    for lane in range(8):
        a_codes |= idx[lane::8] << np.uint32(4 * lane)
    x64 = o.decode(a_codes, a_book, m * k, group).reshape(m, k).astype(np.float64)
    plan = (2, m, n, k, group, 16, 0, 0)
    assert vqdev.path_name(plan) == "onehot-mfma"
    say("cancellation onehot-mfma packed", k, eps)
    out, status = run_plan(vqdev, plan, (a_codes, a_book.reshape(-1), codes, book.reshape(-1)),
                           4 * m * n, np.float32)
    assert status == 0
    ref, st = oracle.matmul(a_codes, a_book, codes, book, m, n, k, group, 0)
    assert st == 0
    _report("onehot-mfma packed", out.reshape(m, n), x64 @ w64, ref, _onehot_bound(x64, w64, k))

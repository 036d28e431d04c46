"""The dense-activation product (ack_vq_matmul_dense): op 2's plan with the
activations handed over as dense float32 instead of a vq4 image. The General
path must equal the oracle's op-2 loop with A read from x bit for bit; the
factorised paths (m = 1, 2..8, >= 32) must agree with the float64 product
within 1e-5 max-rel and with the oracle within FP32 rounding."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import binned_path, onehot_auto, say, small_auto_path

pytestmark = pytest.mark.gpu


def _weight(rng, shape, group, scale=0.02):
    from alelyon_compute_kit import vq
    w = (rng.standard_normal(shape) * scale).astype(np.float32)
    return vq.encode(w, vq.fit_codebook(w, group=group), group=group)


def _check(vqdev, oracle, x, w, transpose_a, transpose_b, path, tol=1e-5, binned=None):
    """`path` is the automatic choice; "small" stands for that of up to 8 rows
    (gemv-direct up to 2^25 weights, else the bin kernels). Where the choice is
    gemv-direct the product is also checked under the test policy, on the bin
    kernel `binned` names (by default gemv-pairs for m = 1, else gemv-rows)."""
    from alelyon_compute_kit import vq
    m, n, k, flags = vq.VQDevice.dense_geometry(x, w, transpose_a, transpose_b)
    if path == "small":
        path = _dense_onehot(m, n, k, w.group, flags) or small_auto_path(m, n, k)
    if path == "gemv-direct":
        vqdev.device.set_policy(2)
        try:
            label = binned or binned_path(m)
            say("dense matmul", label, "(test policy)", m, n, k, w.group, flags)
            _check_run(vqdev, oracle, x, w, transpose_a, transpose_b, label, tol)
        finally:
            vqdev.device.set_policy(0)
    words = (2, m, n, k, w.group, 16, flags, 0)
    assert vqdev.dense_path_name(words) == path
    say("dense matmul", path, m, n, k, w.group, flags)
    return _check_run(vqdev, oracle, x, w, transpose_a, transpose_b, path, tol)


def _dense_onehot(m, n, k, group, flags):
    """"onehot-mfma" where the automatic dense choice takes it: from 64 rows,
    or from 9 with B of at least 2^20 values; None otherwise."""
    return "onehot-mfma" if onehot_auto(m, n, k, group, flags, dense=True) else None


def _dense_x2(m, n, group):
    """Whether the dense one-hot product takes x's bf16 planes: its grid of
    128-row blocks has at least 256 blocks."""
    return (n // (8 * group)) * ((m + 127) // 128) >= 256


def _check_run(vqdev, oracle, x, w, transpose_a, transpose_b, path, tol):
    from alelyon_compute_kit import vq
    from oracle import vq4_numpy as o
    m, n, k, flags = vq.VQDevice.dense_geometry(x, w, transpose_a, transpose_b)
    y = vqdev.matmul_dense(x, w, transpose_a=transpose_a, transpose_b=transpose_b)
    ref, status = oracle.matmul_dense(x, w.codes, w.codebook, m, n, k, w.group, flags)
    assert status == 0
    if path == "general":
        np.testing.assert_array_equal(y.view(np.uint32), ref.view(np.uint32))
    b = w.decode()
    exact = o.matmul64(x, b, transpose_a, transpose_b)
    assert o.max_rel(y, exact) <= tol
    return y


@pytest.mark.parametrize("group", [8, 16, 32])
@pytest.mark.parametrize("m", [1, 2, 5, 8])
def test_dense_gemv_paths(vqdev, oracle, group, m):
    rng = np.random.default_rng(m * 100 + group)
    k, n = 1536, 8 * group * 40            # 40 word columns: one full tile and a ragged one
    w = _weight(rng, (k, n), group)
    x = rng.standard_normal((m, k)).astype(np.float32)
    _check(vqdev, oracle, x, w, False, False, "small")


@pytest.mark.parametrize("m,k,group", [(1, 20000, 16), (4, 20000, 8), (3, 700, 32),
                                       (32, 4096, 16), (19, 3072, 8)])
def test_dense_gemv_split_and_ragged_k(vqdev, oracle, m, k, group):
    rng = np.random.default_rng(k + m)
    n = 8 * group * 32
    w = _weight(rng, (k, n), group)
    x = rng.standard_normal((m, k)).astype(np.float32)
    _check(vqdev, oracle, x, w, False, False, "small")


def test_dense_gemv_transposed_activations(vqdev, oracle):
    rng = np.random.default_rng(5)
    w = _weight(rng, (1024, 8 * 16 * 32), 16)
    x = rng.standard_normal((1024, 6)).astype(np.float32)     # stored k x m
    _check(vqdev, oracle, x, w, True, False, "small")


def _rows_within(y, exact, tol=1e-5):
    """Each row against its own largest magnitude."""
    from oracle import vq4_numpy as o
    for r in range(exact.shape[0]):
        if np.any(exact[r]):
            assert o.max_rel(y[r], exact[r]) <= tol, f"row {r}"
        else:
            assert not np.any(y[r]), f"row {r}"


def test_dense_gemv_outliers_and_zero_rows(vqdev, oracle):
    rng = np.random.default_rng(6)
    w = _weight(rng, (2048, 8 * 16 * 32), 16)
    x = rng.standard_normal((4, 2048)).astype(np.float32)
    x[1] = 0.0                                              # an all-zero row
    x[2, 7] = 30.0                                          # one outlier in a N(0,1) row
    y = _check(vqdev, oracle, x, w, False, False, "small")
    _rows_within(y, x.astype(np.float64) @ w.decode().astype(np.float64))
    zero = np.zeros((1, 2048), np.float32)
    y = vqdev.matmul_dense(zero, w)
    assert not np.any(y)


@pytest.mark.parametrize("m", [1, 4, 8])
@pytest.mark.parametrize("k", [4096, 14336])
def test_dense_gemv_outlier_per_row(vqdev, oracle, m, k):
    """N(0,1) rows with one activation of 30 each, at config 3's k and at
    config 4's 14336 (several integer windows)."""
    rng = np.random.default_rng(k + m)
    w = _weight(rng, (k, 2048), 16)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[np.arange(m), rng.integers(0, k, m)] = 30.0
    y = _check(vqdev, oracle, x, w, False, False, "small")
    _rows_within(y, x.astype(np.float64) @ w.decode().astype(np.float64))


def test_dense_gemv_rows_of_very_different_magnitude(vqdev, oracle):
    """Rows 1e-6, 1, 30 and 1e-30 in scale in one product: each row has its
    own fixed-point scale, so each keeps the 1e-5 bar against its own
    largest output (one scale from the largest row would zero the others)."""
    rng = np.random.default_rng(61)
    w = _weight(rng, (4096, 4096), 16)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    x *= np.array([[1e-6], [1.0], [30.0], [1e-30]], np.float32)
    y = _check(vqdev, oracle, x, w, False, False, "small")
    _rows_within(y, x.astype(np.float64) @ w.decode().astype(np.float64))


@pytest.mark.parametrize("m", [1, 3])
def test_dense_gemv_tiny_activations(vqdev, oracle, m):
    """Activations summing to far below 2^-96 per window (the fixed-point
    shift passes 126; the scale back is taken in two exact steps): the
    results are those of the float64 product, not zero."""
    rng = np.random.default_rng(62 + m)
    w = _weight(rng, (2048, 4096), 16, scale=1.0)
    x = (rng.standard_normal((m, 2048)) * 1e-33).astype(np.float32)
    y = _check(vqdev, oracle, x, w, False, False, "small")
    assert np.abs(y).max() > 0
    _rows_within(y, x.astype(np.float64) @ w.decode().astype(np.float64))


@pytest.mark.parametrize("group", [8, 16, 32])
def test_dense_large_m_every_group(vqdev, oracle, group):
    """Dense rows of m >= 64 take onehot-mfma in every group, group 8 included
    (dense A has no groups to straddle), by default and under the test policy
    (no bin kernel serves m >= 64)."""
    rng = np.random.default_rng(group + 1)
    m, k, n = 128, 512, 8 * group * 6
    w = _weight(rng, (k, n), group)
    x = rng.standard_normal((m, k)).astype(np.float32)
    _check(vqdev, oracle, x, w, False, False, "onehot-mfma")
    vqdev.device.set_policy(2)
    try:
        say("dense matmul", "onehot-mfma (test policy)", m, n, k, group)
        _check_run(vqdev, oracle, x, w, False, False, "onehot-mfma", 1e-5)
    finally:
        vqdev.device.set_policy(0)


# (m, k, n, group): grids of at least 256 blocks of 128 rows (x's bf16 planes,
# 128-row blocks, or 256-row blocks where their grid is as large: 257 rows):
# ragged last row block, group 8, k not a multiple of g
DENSE_X2_SHAPES = [(512, 1024, 4096, 8), (257, 512, 16384, 16), (300, 528, 24576, 32),
                   (384, 1040, 12288, 16)]


@pytest.mark.parametrize("m,k,n,group", DENSE_X2_SHAPES)
def test_dense_onehot_mfma_128_row_blocks(vqdev, oracle, m, k, n, group):
    """Dense activations on large grids: x split once into bf16 planes, read
    by 128-row blocks (each one-hot fragment feeding the 32-row blocks of a
    wave); every row within 1e-5 of the float64 product against its own
    largest output, rows of very different magnitude."""
    assert _dense_x2(m, n, group)
    rng = np.random.default_rng(m + k + n + group)
    w = _weight(rng, (k, n), group)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1] *= 1e-6
    x[130] *= 1e20
    x[m - 1] *= 1e-30
    y = _check(vqdev, oracle, x, w, False, False, "onehot-mfma")
    _rows_within(y, x.astype(np.float64) @ w.decode().astype(np.float64))


# (m, k, n, group): grids of at least 256 blocks of 256 rows (x's bf16 planes
# read by 256-row blocks, each wave 64 rows): benchmark config 4's forward with
# dense activations at full size, group 8, and a ragged last block (rows
# 1024 .. 1099: one wave full, one partly past m, two wholly past it)
DENSE_256_SHAPES = [(2048, 4096, 14336, 32), (1024, 1024, 7168, 8), (1100, 512, 16384, 16)]


@pytest.mark.parametrize("m,k,n,group", DENSE_256_SHAPES)
def test_dense_onehot_mfma_256_row_blocks(vqdev, m, k, n, group):
    """Dense activations on 256-row blocks at full size: every row within
    1e-5 of the float64 product against its own largest output, with rows of
    very different magnitude in several blocks and waves."""
    assert (n // (8 * group)) * ((m + 255) // 256) >= 256
    rng = np.random.default_rng(m + k + n + group)
    w = _weight(rng, (k, n), group)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1] *= 1e-6
    x[200] *= 1e20
    x[700] *= 1e-20
    x[m - 1] *= 1e-30
    words = (2, m, n, k, group, 16, 0, 0)
    assert vqdev.dense_path_name(words) == "onehot-mfma"
    say("dense matmul 256-row blocks", m, n, k, group)
    y, status = _run_status(vqdev, x, w, words)
    assert status == 0
    _rows_within(y, x.astype(np.float64) @ w.decode().astype(np.float64))


def _run_status(vqdev, x, w, words):
    """One dense product through the resident entry: (output, status word)."""
    m, n = words[1], words[2]
    device = vqdev.device
    bufs = [device.buffer(a.nbytes) for a in (x, w.codes, w.codebook)]
    out, status = device.buffer(4 * m * n), device.buffer(4)
    try:
        for b_, a in zip(bufs, (x, w.codes, w.codebook)):
            b_.upload(a)
        status.upload(np.zeros(1, np.uint32))
        vqdev.run_dense(words, *bufs, out, status)
        return out.download(np.float32).reshape(m, n), int(status.download(np.uint32)[0])
    finally:
        for b_ in bufs + [out, status]:
            b_.free()


def _small_book(w, group, top=2.0 ** -10):
    """w's image with its book scaled so that every |C_B| <= top."""
    from alelyon_compute_kit import vq
    book = (w.codebook / np.abs(w.codebook).max() * top).astype(np.float32)
    return vq.VQArray(w.shape, group, w.codes, book)


def test_dense_onehot_mfma_activations_near_float_max(vqdev, oracle):
    """Single activations between the largest bf16 (0x1.fep127) and just
    below FLT_MAX: the bf16 split's first term stops at the largest bf16
    instead of rounding to infinity, and the terms are accumulated smallest
    first, so where every code bucket's sum of x stays clear of FLT_MAX the
    output is finite, no status bit is raised and every row is within 1e-5 of
    the float64 product. (A bucket sum within about an ulp of FLT_MAX can
    overflow: the bf16 MFMA aligns its small addends to the largest by
    truncation, so -FLT_MAX plus negative neighbours reaches -2^128. That
    case raises status bit 1.)"""
    rng = np.random.default_rng(77)
    for m, k, n, group in ((64, 256, 1024, 16), (256, 512, 16384, 8)):
        w = _small_book(_weight(rng, (k, n), group, scale=1.0), group)
        x = rng.standard_normal((m, k)).astype(np.float32)
        x[0, 5] = np.float32(3.4e38)                          # past the largest bf16
        x[2, 9] = np.float32(3.402e38)                        # 2^-12 below FLT_MAX
        x[2, 100] = np.float32(-3.39e38)
        x[5, 17] = -np.float32(3.402e38)
        exact = x.astype(np.float64) @ w.decode().astype(np.float64)
        assert np.isfinite(exact).all()
        y = _check(vqdev, oracle, x, w, False, False, "onehot-mfma")
        assert np.isfinite(y).all()
        _rows_within(y, exact)


def test_dense_bucket_sums_past_float_max_raise_status(vqdev):
    """The factorised products sum x per code bucket before applying C_B.
    Where those sums overflow FP32 (a row of activations all near FLT_MAX)
    the result cannot be formed in FP32 even though the shader's running sum
    of x b stays finite: status bit 1 refuses the output, never a silent
    wrong value. onehot-mfma (the bucket sum overflows) and, under the test
    policy, the fixed-point GEMV (the window's L1 overflows, so no int32
    scale exists); gemv-direct (the automatic m = 1 choice) multiplies
    first, like the shader, and returns the finite product."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(78)
    m, k, n, group = 64, 256, 1024, 16
    w = _small_book(_weight(rng, (k, n), group, scale=1.0), group)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0] = np.float32(3.4e38) * np.sign(x[0])
    words = (2, m, n, k, group, 16, 0, 0)
    assert vqdev.dense_path_name(words) == "onehot-mfma"
    say("dense onehot bucket overflow")
    _, status = _run_status(vqdev, x, w, words)
    assert status & 1
    x1 = np.ascontiguousarray(x[:1])
    words1 = (2, 1, n, k, group, 16, 0, 0)
    assert vqdev.dense_path_name(words1) == "gemv-direct"
    say("dense gemv-direct near FLT_MAX")
    y, status = _run_status(vqdev, x1, w, words1)
    exact = x1.astype(np.float64) @ w.decode().astype(np.float64)
    assert status == 0 and o.max_rel(y, exact) <= 1e-5
    vqdev.device.set_policy(2)
    try:
        say("dense gemv-pairs (test policy) L1 overflow")
        _, status = _run_status(vqdev, x1, w, words1)
        assert status & 1
    finally:
        vqdev.device.set_policy(0)


# (m, k, n, group): from 32 rows (k <= 256 m), rows past m in the 64-row block,
# k not a multiple of 8 g, one and several word columns; k split over blocks
# on these small grids (4 ways at 32 x 1024 x 1024 and 200 x 4096 x 4096, 8 at
# the 128-row chunk, 2 at 96 x 1040 x 1024 with a 16-step in the last part,
# 11 at 48 x 4112 x 2048)
DENSE_ONEHOT_SHAPES = [(32, 1024, 1024, 16), (40, 512, 2048, 32), (64, 64, 256, 16),
                       (130, 256, 2048, 16), (200, 4096, 4096, 32), (255, 1040, 768, 16),
                       (128, 4096, 4096, 32), (48, 4112, 2048, 16),
                       (96, 1040, 1024, 32),     # k not a multiple of g (dense rows need not be)
                       (9, 1024, 1024, 16), (20, 4096, 4096, 8), (31, 14336, 4096, 32)]


@pytest.mark.parametrize("m,k,n,group", DENSE_ONEHOT_SHAPES)
def test_dense_onehot_mfma(vqdev, oracle, m, k, n, group):
    """Dense activations on the one-hot MFMA path (64-row blocks on these
    grids, k split over blocks where they are few; from 9 rows with B of at
    least 2^20 values): x split
    into three bf16 terms as it is read; every row within 1e-5 of the float64
    product against its own largest output."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(m + k + n + group)
    w = _weight(rng, (k, n), group)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1] *= 1e-6                               # rows of very different magnitude
    if m > 3:
        x[3] *= 1e20
    y = _check(vqdev, oracle, x, w, False, False, "onehot-mfma")
    _rows_within(y, x.astype(np.float64) @ w.decode().astype(np.float64))


def test_dense_onehot_mfma_nonfinite_activation(vqdev):
    """A NaN or Inf activation reaches every output of its row: status bit 1."""
    from alelyon_compute_kit import vq
    rng = np.random.default_rng(5)
    m, k, n, group = 64, 512, 1024, 16
    w = _weight(rng, (k, n), group)
    for bad in (np.nan, np.inf):
        x = rng.standard_normal((m, k)).astype(np.float32)
        x[7, 100] = bad
        words = (2, m, n, k, group, 16, 0, 0)
        assert vqdev.dense_path_name(words) == "onehot-mfma"
        device = vqdev.device
        bufs = [device.buffer(a.nbytes) for a in (x, w.codes, w.codebook)]
        out, status = device.buffer(4 * m * n), device.buffer(4)
        try:
            for b_, a in zip(bufs, (x, w.codes, w.codebook)):
                b_.upload(a)
            status.upload(np.zeros(1, np.uint32))
            say("dense onehot nonfinite", bad)
            vqdev.run_dense(words, *bufs, out, status)
            assert int(status.download(np.uint32)[0]) == 1
            y = out.download(np.float32).reshape(m, n)
            assert not np.isfinite(y[7]).any() and np.isfinite(np.delete(y, 7, 0)).all()
        finally:
            for b_ in bufs + [out, status]:
                b_.free()


@pytest.mark.parametrize("m,n,k,ta,tb", [(3, 40, 100, False, True), (20, 64, 48, True, True),
                                         (17, 130, 96, False, False), (9, 200, 64, True, False)])
def test_dense_general_is_bit_exact(vqdev, oracle, m, n, k, ta, tb):
    rng = np.random.default_rng(m + n + k)
    w = _weight(rng, (n, k) if tb else (k, n), 16)
    x = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
    _check(vqdev, oracle, x, w, ta, tb, "general")


def test_dense_refusals_and_status(vqdev):
    from alelyon_compute_kit import ack, vq
    rng = np.random.default_rng(9)
    w = _weight(rng, (256, 256), 16)
    with pytest.raises(ValueError):
        vqdev.matmul_dense(np.ones((2, 100), np.float32), w)       # inner sizes differ
    with pytest.raises(ValueError):
        vqdev.matmul_dense(np.full((1, 256), np.nan, np.float32), w)
    with pytest.raises(ValueError):
        vqdev.matmul_dense(np.ones((1, 256), np.float32), w, transpose_b=1)
    device = vqdev.device
    x = device.buffer(256 * 4)
    codes, book = device.buffer(w.codes.nbytes), device.buffer(w.codebook.nbytes)
    out, status = device.buffer(256 * 4), device.buffer(4)
    try:
        xs = np.ones(256, np.float32)
        xs[3] = np.inf
        x.upload(xs)
        codes.upload(w.codes)
        book.upload(w.codebook)
        status.upload(np.zeros(1, np.uint32))
        words = (2, 1, 256, 256, 16, 16, 0, 0)
        vqdev.run_dense(words, x, codes, book, out, status)
        assert int(status.download(np.uint32)[0]) & 1
        with pytest.raises(ack.AckError):
            vqdev.run_dense(words, x, codes, book, x, status)       # output aliases an input
        with pytest.raises(ack.AckError):
            vqdev.run_dense((2, 2, 256, 256, 16, 16, 0, 0), x, codes, book, out, status)
    finally:
        for b in (x, codes, book, out, status):
            b.free()


@pytest.mark.parametrize("m,k", [(8, 136), (8, 264)])
def test_dense_gemv_row_pairs(vqdev, oracle, m, k):
    """A dense product wide enough that its rows alone fill the chip runs, under
    the test policy, each row of x as a pair-bin instance (k need not be a
    multiple of 8 g: dense rows start anywhere), and by default gemv-direct
    (n k at most 2^25); every row keeps the 1e-5 bar against its own largest
    output."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(900 + m)
    group = 8
    n = 8 * group * 32 * (256 // m)            # 256 row instances of whole 32-word tiles
    # (at m = 8, g = 8: n = 65536, the largest dimension a product admits)
    w = _weight(rng, (k, n), group)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1] *= 1e-6                               # rows of very different magnitude
    y = _check(vqdev, oracle, x, w, False, False, "small", binned="gemv-row-pairs")
    exact = o.matmul64(x, w.decode(), False, False)
    for r in range(m):
        assert o.max_rel(y[r], exact[r]) <= 1e-5, r


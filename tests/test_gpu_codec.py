"""GPU parity of encode (op 0), decode (op 1) and AdamW (op 3) against the
shader oracle: bit-exact results and identical status bits."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import image, run_plan, say

pytestmark = pytest.mark.gpu

GROUPS = (8, 16, 32)


def _sizes(group):
    return (1, group - 1, group, 8 * group + 3, 3 * 4096 + 1, 1 << 20)


@pytest.mark.parametrize("group", GROUPS)
def test_decode_bit_exact(vqdev, oracle, group):
    rng = np.random.default_rng(group)
    for m in _sizes(group):
        say("decode", group, m)
        codes, book = image(rng, m, group)
        out, status = run_plan(vqdev, (1, m, 1, 1, group, 16, 0, 0), (codes, book), 4 * m,
                               np.uint32)
        ref, ref_status = oracle.decode(codes, book, m, group)
        np.testing.assert_array_equal(out, ref.view(np.uint32))
        assert status == ref_status == 0


def test_decode_copies_nan_bits_and_reports_them(vqdev, oracle):
    rng = np.random.default_rng(5)
    codes, book = image(rng, 1000, 16)
    book.view(np.uint32)[:, 3] = 0x7fc0abcd
    say("decode nan payload")
    out, status = run_plan(vqdev, (1, 1000, 1, 1, 16, 16, 0, 0), (codes, book), 4000, np.uint32)
    ref, ref_status = oracle.decode(codes, book, 1000, 16)
    np.testing.assert_array_equal(out, ref.view(np.uint32))
    assert status == ref_status == 1


def test_decode_through_vqdevice(vqdev):
    from alelyon_compute_kit import vq
    rng = np.random.default_rng(6)
    for shape, group in (((256, 256), 16), ((3, 5), 8), ((7, 11, 13), 32)):
        say("VQDevice.decode", shape, group)
        codes, book = image(rng, int(np.prod(shape)), group)
        img = vq.VQArray(shape, group, codes, book)
        np.testing.assert_array_equal(vqdev.decode(img), img.decode())


@pytest.mark.parametrize("group", GROUPS)
def test_encode_bit_exact(vqdev, oracle, group):
    rng = np.random.default_rng(100 + group)
    for m in _sizes(group):
        say("encode", group, m)
        x = rng.standard_normal(m).astype(np.float32)
        book = rng.standard_normal((16, group)).astype(np.float32)
        words = -(-(-(-m // group)) // 8)
        out, status = run_plan(vqdev, (0, m, 1, 1, group, 16, 0, 0), (x, book), 4 * words,
                               np.uint32)
        ref, ref_status = oracle.encode(x, book, group)
        np.testing.assert_array_equal(out, ref)
        assert status == ref_status == 0


@pytest.mark.parametrize("group", GROUPS)
def test_encode_near_ties_and_duplicates(vqdev, oracle, group):
    """Values on Voronoi boundaries and duplicate entries: the lowest index
    wins exactly as the FP32 shader decides."""
    rng = np.random.default_rng(200 + group)
    book = rng.standard_normal((16, group)).astype(np.float32)
    book[9] = book[3] + np.float32(2.0)
    book[12] = book[5]
    mid = book[3] + np.float32(1.0)
    x = np.concatenate([np.tile(mid, 50), np.tile(book[5], 30),
                        rng.standard_normal(group * 40).astype(np.float32) * 0.01])
    x = x.astype(np.float32)
    say("encode ties", group)
    words = -(-(x.size // group) // 8)
    out, status = run_plan(vqdev, (0, x.size, 1, 1, group, 16, 0, 0), (x, book), 4 * words,
                           np.uint32)
    ref, _ = oracle.encode(x, book, group)
    np.testing.assert_array_equal(out, ref)


@pytest.mark.parametrize("group", GROUPS)
def test_encode_screen_margins(vqdev, oracle, group):
    """The kernel ranks codes by |c|^2 - 2 x.c and keeps that ranking only
    when a rounding bound proves it equals the shader's FP32 argmin. Vectors
    placed at offsets from 1e-9 to 1e-2 on either side of a boundary between
    two codes, at scales from subnormal squares to just past the 2^120 cut,
    and a book too large for the screen must all encode bit-exactly."""
    rng = np.random.default_rng(300 + group)
    base = rng.standard_normal((16, group)).astype(np.float32)
    offsets = np.concatenate([-np.logspace(-9, -2, 29), [0.0], np.logspace(-9, -2, 29)])
    pairs = [(a, b) for a in range(16) for b in range(16) if a < b][::7]
    for scale in (2.0 ** -70, 2.0 ** -60, 2.0 ** -20, 1.0, 2.0 ** 40, 2.0 ** 57, 2.0 ** 58, 2.0 ** 59):
        book = (base * np.float32(scale)).astype(np.float32)
        rows = []
        for a, b in pairs:
            mid = (book[a].astype(np.float64) + book[b]) / 2
            step = book[a].astype(np.float64) - book[b]
            rows.append(mid[None, :] + offsets[:, None] * step[None, :])
        x = np.concatenate(rows).astype(np.float32).reshape(-1)
        # random vectors at the same scale fill out the waves
        x = np.concatenate([x, (rng.standard_normal(64 * group) * scale).astype(np.float32)])
        say("encode screen", group, scale)
        words = -(-(x.size // group) // 8)
        out, status = run_plan(vqdev, (0, x.size, 1, 1, group, 16, 0, 0), (x, book), 4 * words,
                               np.uint32)
        ref, ref_status = oracle.encode(x, book, group)
        np.testing.assert_array_equal(out, ref)
        assert status == ref_status
    # one entry with |c|^2 >= 2^120 turns the screen off for the whole book
    book = base.copy()
    book[7] = np.float32(2.0 ** 61)
    x = rng.standard_normal(200 * group).astype(np.float32)
    say("encode screen off", group)
    words = -(-(x.size // group) // 8)
    out, status = run_plan(vqdev, (0, x.size, 1, 1, group, 16, 0, 0), (x, book), 4 * words,
                           np.uint32)
    ref, ref_status = oracle.encode(x, book, group)
    np.testing.assert_array_equal(out, ref)
    assert status == ref_status


def test_encode_status_bits(vqdev, oracle):
    book = np.zeros((16, 8), np.float32)
    for name, x in (("nan", np.array([1, 2, np.nan, 4, 5, 6, 7, 8, 9], np.float32)),
                    ("overflow", np.array([3e19] * 9, np.float32))):
        say("encode status", name)
        out, status = run_plan(vqdev, (0, 9, 1, 1, 8, 16, 0, 0), (x, book), 4, np.uint32)
        ref, ref_status = oracle.encode(x, book, 8)
        assert status == ref_status == 1
        np.testing.assert_array_equal(out, ref)


@pytest.mark.parametrize("group", GROUPS)
def test_encode_nonfinite_inside_whole_waves(vqdev, oracle, group):
    """NaN, +-Inf and a value whose squared distance overflows, placed inside
    runs of 64 whole vectors (the matrix-core screen's waves): the same codes
    and status bit as the shader, and the vectors around them unaffected."""
    rng = np.random.default_rng(400 + group)
    x = rng.standard_normal(4096 * group).astype(np.float32)
    book = rng.standard_normal((16, group)).astype(np.float32)
    x[5] = np.nan
    x[1000 * group + 3] = np.inf
    x[2000 * group + group - 1] = -np.inf
    x[3000 * group] = np.float32(3e19)
    say("encode nonfinite", group)
    words = -(-(x.size // group) // 8)
    out, status = run_plan(vqdev, (0, x.size, 1, 1, group, 16, 0, 0), (x, book), 4 * words,
                           np.uint32)
    ref, ref_status = oracle.encode(x, book, group)
    np.testing.assert_array_equal(out, ref)
    assert status == ref_status == 1


def test_encode_through_vqdevice_matches_cpu_image(vqdev):
    """benchmark config 1: the GPU encode of the fitted 256x256 weight gives
    the reference's 3,128-byte image."""
    from alelyon_compute_kit import vq
    from conftest import golden
    g = golden("config1.npz")
    book = vq.fit_codebook(g["w"], group=16)
    say("config1 encode")
    img = vqdev.encode(g["w"], book, group=16)
    assert img.to_bytes() == g["w_image"].tobytes()


@pytest.mark.parametrize("op", [0, 1])
def test_batched_codec(vqdev, oracle, op):
    rng = np.random.default_rng(300 + op)
    group, m, count = 16, 1000, 5
    words = -(-(-(-m // group)) // 8)
    if op == 0:
        xs = rng.standard_normal((count, m)).astype(np.float32)
        books = rng.standard_normal((count, 16, group)).astype(np.float32)
        say("batch encode", count)
        out, status = run_plan(vqdev, (0, m, 1, 1, group, 16, 0, 0), (xs, books),
                               4 * words * count, np.uint32, count=count)
        for i in range(count):
            ref, _ = oracle.encode(xs[i], books[i], group)
            np.testing.assert_array_equal(out[i * words:(i + 1) * words], ref)
    else:
        pairs = [image(rng, m, group) for _ in range(count)]
        codes = np.concatenate([c for c, _ in pairs])
        books = np.concatenate([b for _, b in pairs])
        say("batch decode", count)
        out, status = run_plan(vqdev, (1, m, 1, 1, group, 16, 0, 0), (codes, books),
                               4 * m * count, np.uint32, count=count)
        for i, (c, b) in enumerate(pairs):
            ref, _ = oracle.decode(c, b, m, group)
            np.testing.assert_array_equal(out[i * m:(i + 1) * m], ref.view(np.uint32))
    assert status == 0


@pytest.mark.parametrize("group", GROUPS)
@pytest.mark.parametrize("extra", [8, 9])
def test_batched_encode_whole_waves(vqdev, oracle, group, extra):
    """Batched encode over instances of three whole 64-vector waves and a
    tail: the matrix-core screen per instance. With an odd length the
    instances after the first start off a 16-byte boundary and take the
    per-lane screen; the codes are the shader's either way."""
    rng = np.random.default_rng(600 + group + extra)
    m, count = 64 * group * 3 + extra, 4
    words = -(-(-(-m // group)) // 8)
    xs = rng.standard_normal((count, m)).astype(np.float32)
    books = rng.standard_normal((count, 16, group)).astype(np.float32)
    say("batch encode waves", group, m)
    out, status = run_plan(vqdev, (0, m, 1, 1, group, 16, 0, 0), (xs, books),
                           4 * words * count, np.uint32, count=count)
    assert status == 0
    for i in range(count):
        ref, _ = oracle.encode(xs[i], books[i], group)
        np.testing.assert_array_equal(out[i * words:(i + 1) * words], ref)


def _adamw_case(rng, count, group, variance_sign=1.0):
    states = [image(rng, count, group, scale) for scale in (0.05, 1e-2, 1e-4, 1e-2)]
    books = [b for _, b in states]
    books[2] = np.abs(books[2]) * variance_sign
    codes4 = np.concatenate([c for c, _ in states])
    books4 = np.concatenate([b.reshape(-1) for b in books]).astype(np.float32)
    return codes4, books4


@pytest.mark.parametrize("group", GROUPS)
def test_adamw_bit_exact(vqdev, oracle, group):
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(400 + group)
    for count in (1, group + 1, 10007, 1 << 20):
        say("adamw", group, count)
        codes4, books4 = _adamw_case(rng, count, group)
        coeff = o.adamw_coefficients(1e-3, 0.9, 0.999, 1e-8, 0.01, 7)
        out, status = run_plan(vqdev, (3, count, 1, 1, group, 16, 0, 0),
                               (codes4, books4, coeff), 12 * count, np.uint32)
        ref, ref_status = oracle.adamw(codes4, books4, coeff, count, group)
        np.testing.assert_array_equal(out, ref.view(np.uint32))
        assert status == ref_status == 0


@pytest.mark.parametrize("group", [8, 16])
def test_adamw_quads_tail_and_overflowing_entry(vqdev, oracle, group):
    """Op 3 on 16-byte quads with a partial last vector (m = 1000 g + 4): a
    gradient entry whose last component squares past FLT_MAX, so V' of that
    component alone is infinite. Read only by the last vector, whose element
    stops four components in, it raises nothing; read by a whole vector it
    raises bit 1. Outputs and status as the shader's."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(500 + group)
    count = 1000 * group + 4
    vectors = -(-count // group)
    words = -(-vectors // 8)
    coeff = o.adamw_coefficients(1e-3, 0.9, 0.999, 1e-8, 0.01, 3)
    codes4, books4 = _adamw_case(rng, count, group)
    books4 = books4.copy()
    books4[(48 + 15) * group + group - 1] = np.float32(3e19)
    grad_idx = o.unpack_indices(codes4[3 * words:], vectors) % 15
    for name, where, expect in (("unused but by the tail", vectors - 1, 0),
                                ("used by a whole vector", vectors // 2, 1)):
        idx = grad_idx.copy()
        idx[where] = 15
        c4 = codes4.copy()
        c4[3 * words:] = o.pack_indices(idx.astype(np.int64))
        say("adamw quads", group, name)
        out, status = run_plan(vqdev, (3, count, 1, 1, group, 16, 0, 0), (c4, books4, coeff),
                               12 * count, np.uint32)
        ref, ref_status = oracle.adamw(c4, books4, coeff, count, group)
        np.testing.assert_array_equal(out, ref.view(np.uint32))
        assert status == ref_status == expect


def test_adamw_status_bits(vqdev, oracle):
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(9)
    codes4, books4 = _adamw_case(rng, 64, 8)
    good = o.adamw_coefficients(1e-3, 0.9, 0.999, 1e-8, 0.0, 1)
    cases = []
    bad = good.copy()
    bad[3] = np.nan
    cases.append(("nonfinite coefficient", codes4, books4, bad))
    bad = good.copy()
    bad[1] = 1.0
    cases.append(("beta1 domain", codes4, books4, bad))
    neg = _adamw_case(rng, 64, 8, variance_sign=-1.0)
    cases.append(("negative variance", neg[0], neg[1], good))
    for name, c4, b4, coeff in cases:
        say("adamw status", name)
        _, status = run_plan(vqdev, (3, 64, 1, 1, 8, 16, 0, 0), (c4, b4, coeff), 12 * 64,
                             np.uint32)
        _, ref_status = oracle.adamw(c4, b4, coeff, 64, 8)
        assert status == ref_status != 0

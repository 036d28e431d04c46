"""Pins for the shader oracle (oracle/vq4_oracle.c), host only.

The reference runs no test of vq4.comp, so the oracle is checked against
what the mathematics fixes: decode is a gather; encode is an FP32 argmin that
a brute-force numpy float32 loop reproduces and that agrees with the
reference's float64 CPU encode except at near-ties; matmul is the sequential
FP32 sum (brute force on tiny inputs) and within FP32 rounding of a float64
GEMM of the decoded operands; AdamW is the shader's FP32 sequence (numpy
float32 step by step) and within rounding of float64 arithmetic. Each check
has a planted-mistake control that must fail it.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden


def _image(rng, m, group):
    from oracle import vq4_numpy as o
    codes = o.pack_indices(rng.integers(0, 16, -(-m // group)))
    book = rng.standard_normal((16, group)).astype(np.float32)
    return codes, book


def test_decode_is_a_bit_exact_gather(oracle):
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(0)
    for group in (8, 16, 32):
        for m in (1, group + 3, 1000):
            codes, book = _image(rng, m, group)
            book.view(np.uint32)[2, 1] = 0x7fc01234      # a NaN payload survives the copy
            out, status = oracle.decode(codes, book, m, group)
            ref = o.decode(codes, book, m, group)
            np.testing.assert_array_equal(out.view(np.uint32), ref.view(np.uint32))
            assert status == 1                           # the sweep saw the NaN


def _encode_f32_bruteforce(x, book, group):
    """vq4.comp:118-144 with numpy float32 scalars."""
    from oracle import vq4_numpy as o
    f = np.float32
    vectors = -(-x.size // group)
    idx = []
    for v in range(vectors):
        start = v * group
        valid = min(group, x.size - start)
        best, sel = f(np.inf), 0
        for code in range(16):
            d = f(0)
            for j in range(valid):
                delta = f(x[start + j]) - f(book[code, j])
                d = f(d + f(delta * delta))
            if d < best:
                best, sel = d, code
        idx.append(sel)
    return o.pack_indices(idx)


def test_encode_matches_a_float32_brute_force(oracle):
    rng = np.random.default_rng(1)
    for group in (8, 16, 32):
        for m in (1, group - 1, 8 * group + 5):
            x = rng.standard_normal(m).astype(np.float32)
            book = rng.standard_normal((16, group)).astype(np.float32)
            codes, status = oracle.encode(x, book, group)
            np.testing.assert_array_equal(codes, _encode_f32_bruteforce(x, book, group))
            assert status == 0


def test_encode_agrees_with_the_reference_cpu_encode_except_near_ties(oracle):
    from oracle import vq4_numpy as o
    g = golden("encode_cpu.npz")
    disagreements = 0
    for i in range(int(g["count"])):
        tie_case = i % 7 == 6          # each group's seventh case is built from near-ties
        x, book, group = g[f"c{i}_x"], g[f"c{i}_book"], int(g[f"c{i}_group"])
        codes, status = oracle.encode(x, book, group)
        assert status == 0
        n = -(-x.size // group)
        ours, ref = o.unpack_indices(codes, n), o.unpack_indices(g[f"c{i}_codes"], n)
        for v in np.nonzero(ours != ref)[0]:
            seg = x[v * group:(v + 1) * group].astype(np.float64)
            d = ((seg[None, :] - book[:, :seg.size].astype(np.float64)) ** 2).sum(1)
            assert abs(d[ours[v]] - d[ref[v]]) <= 1e-5 * d[ref[v]] + 1e-30
            disagreements += not tie_case
    assert disagreements <= 2


def test_encode_status_bits(oracle):
    x = np.ones(16, np.float32)
    book = np.zeros((16, 8), np.float32)
    assert oracle.encode(x, book, 8)[1] == 0
    x[3] = np.nan
    assert oracle.encode(x, book, 8)[1] == 1
    x[3] = 3e19                                  # (x - c)^2 overflows to inf
    assert oracle.encode(x, book, 8)[1] == 1
    book[15, 7] = np.inf
    assert oracle.encode(np.ones(16, np.float32), book, 8)[1] == 1


def _operands(rng, m, n, k, group, flags):
    a_shape = (k, m) if flags & 1 else (m, k)
    b_shape = (n, k) if flags & 2 else (k, n)
    a_codes, a_book = _image(rng, m * k, group)
    b_codes, b_book = _image(rng, k * n, group)
    return a_codes, a_book, b_codes, b_book, a_shape, b_shape


def _dense(codes, book, shape, group):
    from oracle import vq4_numpy as o
    return o.decode(codes, book, int(np.prod(shape)), group).reshape(shape)


@pytest.mark.parametrize("flags", [0, 1, 2, 3])
def test_matmul_is_the_sequential_float32_sum(oracle, flags):
    rng = np.random.default_rng(2 + flags)
    m, n, k, group = 3, 5, 7, 8                  # groups straddle every row
    a_codes, a_book, b_codes, b_book, a_shape, b_shape = _operands(rng, m, n, k, group, flags)
    out, status = oracle.matmul(a_codes, a_book, b_codes, b_book, m, n, k, group, flags)
    a = _dense(a_codes, a_book, a_shape, group)
    b = _dense(b_codes, b_book, b_shape, group)
    a = a.T if flags & 1 else a
    b = b.T if flags & 2 else b
    f = np.float32
    for r in range(m):
        for c in range(n):
            t = f(0)
            for i in range(k):
                t = f(t + f(a[r, i] * b[i, c]))
            assert out[r, c].view(np.uint32) == t.view(np.uint32)
    assert status == 0


@pytest.mark.parametrize("flags", [0, 1, 2, 3])
def test_matmul_within_float32_rounding_of_float64(oracle, flags):
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(10 + flags)
    m, n, k, group = 37, 53, 96, 16
    a_codes, a_book, b_codes, b_book, a_shape, b_shape = _operands(rng, m, n, k, group, flags)
    out, _ = oracle.matmul(a_codes, a_book, b_codes, b_book, m, n, k, group, flags)
    a = _dense(a_codes, a_book, a_shape, group)
    b = _dense(b_codes, b_book, b_shape, group)
    ref = o.matmul64(a, b, bool(flags & 1), bool(flags & 2))
    assert o.max_rel(out, ref) <= 1e-5
    # planted mistake: the other transpose of B must fail the same bound
    wrong = o.matmul64(a, b.reshape(b.shape[::-1]), bool(flags & 1), not flags & 2)
    assert o.max_rel(out, wrong) > 1e-3


def test_matmul_status_on_overflow(oracle):
    from oracle import vq4_numpy as o
    codes = o.pack_indices(np.zeros(4, np.int64))
    book = np.full((16, 8), 3e19, np.float32)
    _, status = oracle.matmul(codes, book, codes, book, 4, 4, 8, 8, 0)
    assert status == 1


@pytest.mark.parametrize("flags", [0, 1, 2, 3])
def test_dense_matmul_reduces_to_op2_on_decoded_activations(oracle, flags):
    """The dense-activation product's oracle is op 2's loop with A read from x:
    fed x = decode(A) it must equal the op-2 oracle bit for bit, and a dense x
    that no image can hold must match the sequential float32 sum."""
    rng = np.random.default_rng(40 + flags)
    m, n, k, group = 5, 24, 13, 8
    a_codes, a_book, b_codes, b_book, a_shape, b_shape = _operands(rng, m, n, k, group, flags)
    x = _dense(a_codes, a_book, a_shape, group)
    want, s1 = oracle.matmul(a_codes, a_book, b_codes, b_book, m, n, k, group, flags)
    got, s2 = oracle.matmul_dense(x, b_codes, b_book, m, n, k, group, flags)
    assert s1 == s2 == 0
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    x = rng.standard_normal(a_shape).astype(np.float32)
    got, _ = oracle.matmul_dense(x, b_codes, b_book, m, n, k, group, flags)
    a = x.T if flags & 1 else x
    b = _dense(b_codes, b_book, b_shape, group)
    b = b.T if flags & 2 else b
    f = np.float32
    for r in range(m):
        for c in range(n):
            t = f(0)
            for i in range(k):
                t = f(t + f(a[r, i] * b[i, c]))
            assert got[r, c].view(np.uint32) == t.view(np.uint32)
    x[0, 0] = np.inf                            # a nonfinite activation raises bit 1
    assert oracle.matmul_dense(x, b_codes, b_book, m, n, k, group, flags)[1] == 1


def _adamw_f32(w, m, v, g, c):
    f = np.float32
    nm = f(f(c[1] * m) + f(f(f(1) - c[1]) * g))
    nv = f(f(c[2] * v) + f(f(f(1) - c[2]) * f(g * g)))
    den = f(f(np.sqrt(f(nv / c[6]))) + c[3])
    nw = f(f(w * f(f(1) - f(c[0] * c[4]))) - f(f(c[0] * f(nm / c[5])) / den))
    return nw, nm, nv


def _adamw_inputs(rng, count, group, variance_sign=1.0):
    from oracle import vq4_numpy as o
    states = [_image(rng, count, group) for _ in range(4)]
    books = [b for _, b in states]
    books[2] = np.abs(books[2]) * variance_sign
    codes4 = np.concatenate([c for c, _ in states])
    books4 = np.concatenate([b.reshape(-1) for b in books])
    dense = [o.decode(states[s][0], books[s], count, group) for s in range(4)]
    return codes4, books4, dense


def test_adamw_is_the_shaders_float32_sequence(oracle):
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(4)
    for group in (8, 16, 32):
        count = 301
        codes4, books4, (w, m, v, g) = _adamw_inputs(rng, count, group)
        coeff = o.adamw_coefficients(1e-3, 0.9, 0.999, 1e-8, 0.01, 3)
        out, status = oracle.adamw(codes4, books4, coeff, count, group)
        assert status == 0
        nw, nm, nv = _adamw_f32(w, m, v, g, coeff)
        for got, want in zip(np.split(out, 3), (nw, nm, nv)):
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        ref = o.adamw64(w, m, v, g, coeff)
        for got, want in zip(np.split(out, 3), ref):
            assert o.max_rel(got, want) <= 1e-6
        # planted mistake: no bias correction on the first moment
        wrong = w.astype(np.float64) - 1e-3 * ref[1] / (np.sqrt(ref[2] / coeff[6]) + 1e-8)
        assert o.max_rel(np.split(out, 3)[0] - w, wrong - w) > 1e-3


def test_adamw_status_bits(oracle):
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(5)
    codes4, books4, _ = _adamw_inputs(rng, 64, 8)
    good = o.adamw_coefficients(1e-3, 0.9, 0.999, 1e-8, 0.0, 1)
    assert oracle.adamw(codes4, books4, good, 64, 8)[1] == 0
    bad = good.copy()
    bad[3] = np.nan
    assert oracle.adamw(codes4, books4, bad, 64, 8)[1] == 1
    bad = good.copy()
    bad[1] = 1.0                                      # beta1 outside [0, 1)
    out, status = oracle.adamw(codes4, books4, bad, 64, 8)
    assert status == 4 and np.isnan(out).all()        # nothing written
    codes4, books4, _ = _adamw_inputs(rng, 64, 8, variance_sign=-1.0)
    assert oracle.adamw(codes4, books4, good, 64, 8)[1] & 4


# ---- caller-side helpers of the oracle: seeded payloads and the gradient clip ----

def test_expert_payload_equals_the_reference_initializer():
    """oracle expert_payload (restating expert_bank.py:357-390) against the
    payloads the reference's ExpertBank.initialize_expert wrote
    (tests/golden/expert_payloads.npz): config 2's three seed-7 matrices and
    the weight of a zero-optimizer-state bank; bit for bit."""
    from oracle import vq4_numpy as o
    g = golden("expert_payloads.npz")
    for i in range(3):
        codes, book = o.expert_payload((128, 128), 16, 7, 0, 0, i)
        np.testing.assert_array_equal(codes, g[f"c2_{i}_codes"])
        np.testing.assert_array_equal(book.view(np.uint32), g[f"c2_{i}_book"].view(np.uint32))
    codes, book = o.expert_payload((4, 3), 8, 4, 0, 0, 0)
    np.testing.assert_array_equal(codes, g["h_0_codes"])          # tail nibbles masked
    np.testing.assert_array_equal(book.view(np.uint32), g["h_0_book"].view(np.uint32))
    # planted mistakes: another stream index, or a scale by the column count
    assert not np.array_equal(o.expert_payload((128, 128), 16, 7, 0, 0, 1)[0], g["c2_0_codes"])
    wrong = o.expert_payload((4, 3), 8, 4, 0, 0, 0)[1] * np.float32(np.sqrt(4) / np.sqrt(3))
    assert not np.array_equal(wrong, g["h_0_book"])


def test_clip_scale_closed_forms():
    """clip_scale = min(1, max_norm / (||g||_2 + 1e-6)) on gradients of known
    norm: (3, 4) has norm 5 exactly; a gradient inside the ball is not scaled;
    a zero gradient divides by 1e-6 alone."""
    from oracle import vq4_numpy as o
    g = np.array([[3.0, 4.0]], np.float32)
    assert o.clip_scale(g, 1.0) == 1.0 / (5.0 + 1e-6)
    assert o.clip_scale(g, 10.0) == 1.0
    assert o.clip_scale(np.zeros((2, 2), np.float32), 1e-9) == min(1.0, 1e-9 / 1e-6)
    # 12 x 12 of 0.25: sum of squares 9, norm 3 exactly
    assert o.clip_scale(np.full((12, 12), 0.25, np.float32), 0.3) == 0.3 / (3.0 + 1e-6)
    # planted mistake: the squared norm in place of the norm fails the first case
    assert 1.0 / (25.0 + 1e-6) != o.clip_scale(g, 1.0)


def test_clip_scale_equals_the_reference_harness():
    """clip_scale against the clip the reference harness applied on real
    steps (tests/golden/clip_scale.npz, recorded through
    VulkanExpertHarness.train_step with a host backend): the same norm, and
    the gradient times float32(scale) equal bit for bit to the clipped
    gradient it encoded; the same clipped/unclipped verdict."""
    from oracle import vq4_numpy as o
    g = golden("clip_scale.npz")
    for i in range(int(g["count"])):
        before, after = g[f"c{i}_before"], g[f"c{i}_after"]
        max_norm = float(g[f"c{i}_max_norm"])
        scale = o.clip_scale(before, max_norm)
        assert float(np.linalg.norm(before.astype(np.float64))) == float(g[f"c{i}_norm"])
        assert (scale < 1.0) == bool(g[f"c{i}_clipped"])
        clipped = before * np.float32(scale)
        np.testing.assert_array_equal(clipped.view(np.uint32), after.view(np.uint32))
    # planted mistake: without the 1e-6 the clipped cases differ in their last bits
    i = next(i for i in range(int(g["count"])) if bool(g[f"c{i}_clipped"]))
    before, after = g[f"c{i}_before"], g[f"c{i}_after"]
    norm = float(np.linalg.norm(before.astype(np.float64)))
    wrong = before * np.float32(float(g[f"c{i}_max_norm"]) / norm)
    assert not np.array_equal(wrong.view(np.uint32), after.view(np.uint32))

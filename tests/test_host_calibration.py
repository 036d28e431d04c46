"""CPU encode and fit_codebook (vq.py:154-257): the product's native host
code and the oracle's numpy restatement, both against golden vectors recorded
from the reference, plus the reference's own property tests
(tests/test_fit_codebook_keeps_every_entry.py)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden


def _cases(name):
    g = golden(name)
    for i in range(int(g["count"])):
        case = {k[len(f"c{i}_"):]: v for k, v in g.items() if k.startswith(f"c{i}_")}
        if "values_ref" in case:
            case["values"] = g[f"c{int(case['values_ref'])}_values"]
        yield i, case


def test_product_encode_matches_reference_vectors():
    from alelyon_compute_kit import vq
    for i, c in _cases("encode_cpu.npz"):
        img = vq.encode(c["x"], c["book"], group=int(c["group"]))
        np.testing.assert_array_equal(img.codes, c["codes"], err_msg=f"case {i}")


def test_oracle_encode_matches_reference_vectors():
    from oracle import vq4_numpy as o
    for i, c in _cases("encode_cpu.npz"):
        np.testing.assert_array_equal(o.encode64(c["x"], c["book"], int(c["group"])), c["codes"],
                                      err_msg=f"case {i}")


def test_exact_ties_pick_the_lowest_index():
    from alelyon_compute_kit import vq
    book = np.zeros((16, 8), np.float32)
    book[5] = 2.0
    book[0] = 4.0          # entries 1..4 and 6..15 tie at distance 8*1; entry 1 wins
    book[1:5] = 0.0
    x = np.ones(8, np.float32)
    assert int(vq.encode(x, book, group=8).codes[0]) == 1
    book[1:5] = 2.0        # now entries 1..5 tie at 8: 1 still wins over 5
    assert int(vq.encode(x, book, group=8).codes[0]) == 1


def test_product_fit_matches_reference_vectors():
    from alelyon_compute_kit import vq
    for i, c in _cases("fit_codebook.npz"):
        init = c["init"] if c["init"].size else None
        book = vq.fit_codebook(c["values"], group=int(c["group"]),
                               iterations=int(c["iterations"]),
                               sample_vectors=int(c["sample_vectors"]), init=init)
        np.testing.assert_array_equal(book, c["book"], err_msg=f"case {i}")


def test_oracle_fit_matches_reference_vectors():
    from oracle import vq4_numpy as o
    for i, c in _cases("fit_codebook.npz"):
        init = c["init"] if c["init"].size else None
        book = o.fit_codebook(c["values"], int(c["group"]), int(c["iterations"]),
                              int(c["sample_vectors"]), init)
        np.testing.assert_array_equal(book, c["book"], err_msg=f"case {i}")


@pytest.mark.parametrize("n", [1, 2, 15, 16, 17, 100, 4096, 4097, 8192, 65536, 123457])
def test_linspace_sampling_matches_numpy(n):
    """The sample indices are numpy.linspace(..., dtype=int64): checked through
    a fit whose sample is the identity of its rows."""
    from alelyon_compute_kit import vq
    rows = np.arange(n, dtype=np.float32)
    values = np.repeat(rows, 8)
    book = vq.fit_codebook(values, group=8, iterations=0, sample_vectors=4096)
    sample = np.linspace(0, n - 1, min(n, 4096), dtype=np.int64)
    expected = sample[np.linspace(0, len(sample) - 1, 16, dtype=np.int64)]
    np.testing.assert_array_equal(book[:, 0], expected.astype(np.float32))


DIMS = 16
OCCUPANCY = {
    "even": [64] * 16,
    "eight common, eight rare": [120] * 8 + [8] * 8,
    "skewed geometric": [max(1, int(512 * 0.55 ** i)) for i in range(16)],
    "one dominant, fifteen rare": [900] + [4] * 15,
}


def _sample_of(counts):
    atoms = np.random.default_rng(1).standard_normal((16, DIMS))
    return np.repeat(atoms, counts, axis=0).astype(np.float32)


def _indices(sample, book):
    from alelyon_compute_kit import vq
    codes = vq.encode(sample, book, group=DIMS).codes
    pos = np.arange(len(sample))
    return (codes[pos // 8] >> ((pos % 8) * 4).astype(np.uint32)) & 15


@pytest.mark.parametrize("name", list(OCCUPANCY))
def test_every_entry_is_distinct_and_reachable(name):
    from alelyon_compute_kit import vq
    sample = _sample_of(OCCUPANCY[name])
    book = vq.fit_codebook(sample.reshape(-1), group=DIMS)
    assert len(np.unique(book.round(6), axis=0)) == 16
    assert len(np.unique(_indices(sample, book))) == 16


def test_identical_input_collapses():
    from alelyon_compute_kit import vq
    book = vq.fit_codebook(np.ones((512, DIMS), np.float32).reshape(-1), group=DIMS)
    assert len(np.unique(book.round(6), axis=0)) == 1


def test_oracle_fit_can_fail_the_property_it_guards():
    """Positive control planted in the oracle: the pre-fix loop (no reseed)
    must lose entries on this occupancy, or the test above is vacuous."""
    from oracle import vq4_numpy as o
    sample = _sample_of(OCCUPANCY["one dominant, fifteen rare"])
    book = sample[np.linspace(0, len(sample) - 1, 16, dtype=np.int64)].copy()
    for _ in range(4):
        idx = o.unpack_indices(o.encode64(sample, book, DIMS), len(sample))
        for e in range(16):
            rows = sample[idx == e]
            if len(rows):
                book[e] = rows.mean(axis=0, dtype=np.float64).astype(np.float32)
    assert len(np.unique(book.round(6), axis=0)) < 16


def test_fit_refusals():
    from alelyon_compute_kit import vq
    with pytest.raises(ValueError, match="complete vector"):
        vq.fit_codebook(np.ones(7, np.float32), group=8)
    with pytest.raises(ValueError, match="finite float32"):
        vq.fit_codebook(np.full(16, np.inf, np.float32), group=8)
    with pytest.raises(ValueError, match="iterations"):
        vq.fit_codebook(np.ones(16, np.float32), group=8, iterations=33)
    with pytest.raises(ValueError, match="sample_vectors"):
        vq.fit_codebook(np.ones(16, np.float32), group=8, sample_vectors=15)
    with pytest.raises(ValueError, match="codebook"):
        vq.fit_codebook(np.ones(16, np.float32), group=8, init=np.zeros((16, 16), np.float32))


class Float32Backend:
    """Host backend: AdamW in numpy float32 in the shader's order; CPU encode.
    The same arithmetic the golden steps were recorded with."""

    def encode(self, values, codebook, *, group):
        from alelyon_compute_kit import vq
        return vq.encode(values, codebook, group=group)

    def decode(self, value):
        return value.decode()

    def adamw(self, weight, momentum, variance, gradient, *, lr, beta1, beta2, eps,
              weight_decay, step):
        from oracle import vq4_numpy as o
        f = np.float32
        c = o.adamw_coefficients(lr, beta1, beta2, eps, weight_decay, step)
        w, m, v, g = (s.decode() for s in (weight, momentum, variance, gradient))
        nm = c[1] * m + (f(1) - c[1]) * g
        nv = c[2] * v + (f(1) - c[2]) * (g * g)
        den = np.sqrt(nv / c[6]) + c[3]
        nw = w * (f(1) - c[0] * c[4]) - c[0] * (nm / c[5]) / den
        return nw.astype(np.float32), nm.astype(np.float32), nv.astype(np.float32)


def test_vqadamw_steps_match_the_reference_with_a_host_backend():
    """VQAdamW.step's orchestration -- op-3 scratch, warm-started refit per
    state, re-encode, changed count -- against the reference's own step on the
    same host backend."""
    from alelyon_compute_kit import vq
    g = golden("vqadamw_steps.npz")
    for i in range(3):
        group = int(g[f"s{i}_group"])
        shape = tuple(int(x) for x in g[f"s{i}_shape"])
        weight = vq.VQArray(shape, group, g[f"s{i}_w0_codes"], g[f"s{i}_w0_book"])
        opt = vq.VQAdamW(Float32Backend(), weight, lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
                         weight_decay=0.01)
        for step in range(2):
            grad = vq.VQArray(shape, group, g[f"s{i}_g{step}_codes"], g[f"s{i}_g{step}_book"])
            report = opt.step(grad)
            assert report["changed_weight_values"] == int(g[f"s{i}_changed{step}"])
            for name, state in (("w", opt.weight), ("m", opt.momentum), ("v", opt.variance)):
                np.testing.assert_array_equal(state.codes, g[f"s{i}_{name}{step + 1}_codes"])
                np.testing.assert_array_equal(state.codebook, g[f"s{i}_{name}{step + 1}_book"])


def _review_shape(group, rare_at=-1):
    vectors = 65536 // group
    atoms = np.random.default_rng(1).standard_normal((16, group)).astype(np.float32)
    index = np.insert(np.arange(vectors - 1) % 15, rare_at % vectors, 15)
    return atoms, index


@pytest.mark.parametrize("group,rare_at", [(8, -1), (16, -1), (32, -1), (8, 1)])
def test_zero_gradient_moves_no_weight(group, rare_at):
    """The audit's acceptance test at its shape (65,536 values)."""
    from alelyon_compute_kit import vq
    atoms, index = _review_shape(group, rare_at)
    values = atoms[index].reshape(-1)
    weight = vq.encode(values, atoms, group=group)
    assert np.array_equal(weight.decode(), values)
    zero = vq.VQArray(weight.shape, group, np.zeros_like(weight.codes),
                      np.zeros((16, group), np.float32))
    opt = vq.VQAdamW(Float32Backend(), weight, lr=1e-3, weight_decay=0.0)
    before = opt.weight.decode().copy()
    report = opt.step(zero)
    after = opt.weight.decode()
    assert report["changed_weight_values"] == int((before != after).sum()) == 0
    assert len(np.unique(opt.weight.codebook.round(6), axis=0)) == 16

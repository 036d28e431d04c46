"""fit_codebook on the GPU (ack_vq_fit_codebook, vq.py:182-257): the books must
equal, bit for bit, the reference's own recorded outputs (golden vectors) and
the native host fit -- which those vectors pin -- on inputs chosen to drive
every branch: cold and warm starts, a sample smaller than the tensor, the
whole-tensor keep pass, reseeds of empty entries (many at once from a book of
identical rows), ties, and tails that are not whole vectors."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden
from gpu_util import say

pytestmark = pytest.mark.gpu


def _both(vqdev, values, **kwargs):
    from alelyon_compute_kit import vq
    host = vq.fit_codebook(values, **kwargs)
    dev = vqdev.fit_codebook(values, **kwargs)
    return host, dev


def test_device_fit_matches_reference_vectors(vqdev):
    g = golden("fit_codebook.npz")
    for i in range(int(g["count"])):
        c = {k[len(f"c{i}_"):]: v for k, v in g.items() if k.startswith(f"c{i}_")}
        values = g[f"c{int(c['values_ref'])}_values"] if "values_ref" in c else c["values"]
        init = c["init"] if c["init"].size else None
        say("golden fit case", i, values.size, int(c["group"]))
        book = vqdev.fit_codebook(values, group=int(c["group"]), iterations=int(c["iterations"]),
                                  sample_vectors=int(c["sample_vectors"]), init=init)
        np.testing.assert_array_equal(book, c["book"], err_msg=f"case {i}")


@pytest.mark.parametrize("group", [8, 16, 32])
@pytest.mark.parametrize("vectors,sample,iterations", [(40, 4096, 4), (5000, 4096, 4),
                                                        (70000, 4096, 2), (3000, 16, 7),
                                                        (3, 4096, 4), (20000, 65536, 1),
                                                        (1000, 4096, 0)])
def test_cold_fit_equals_the_host_fit(vqdev, group, vectors, sample, iterations):
    rng = np.random.default_rng(vectors + group)
    values = rng.standard_normal(vectors * group + group // 2).astype(np.float32)
    say("cold fit", group, vectors, sample, iterations)
    host, dev = _both(vqdev, values, group=group, iterations=iterations, sample_vectors=sample)
    np.testing.assert_array_equal(dev, host)


@pytest.mark.parametrize("group", [8, 16, 32])
@pytest.mark.parametrize("spread", [0, 20])
def test_fit_means_exact_in_any_order_or_in_sample_order(vqdev, group, spread):
    """An entry's mean sums its members in sample order (numpy's axis 0). With
    one staging round the device first sums in any order and keeps that only
    when no partial sum can round (values within 53 bits of each other, as
    codebook-built states are); magnitudes spread over 10^spread exceed that
    and take the in-order sum. Both must give the host fit's books; a zero
    book sends the whole sample to one entry (the longest sum)."""
    rng = np.random.default_rng(300 + group + spread)
    vectors = 4096
    scale = 10.0 ** rng.uniform(-spread, 0, vectors * group)
    values = (rng.standard_normal(vectors * group) * scale).astype(np.float32)
    say("fit means", group, spread)
    host, dev = _both(vqdev, values, group=group)
    np.testing.assert_array_equal(dev, host)
    zero = np.zeros((16, group), np.float32)
    host, dev = _both(vqdev, values, group=group, init=zero)
    np.testing.assert_array_equal(dev, host)


@pytest.mark.parametrize("group", [8, 16, 32])
def test_warm_fit_with_the_keep_pass_equals_the_host_fit(vqdev, group):
    """Rare vectors the strided sample misses still select entry 15 of the warm
    book, so the whole-tensor pass keeps it instead of reseeding it."""
    rng = np.random.default_rng(group)
    atoms = rng.standard_normal((16, group)).astype(np.float32)
    vectors = 20000
    index = np.arange(vectors) % 15
    sampled = np.linspace(0, vectors - 1, 4096).astype(np.int64)
    index[np.setdiff1d(np.arange(vectors), sampled)[[500, 9000]]] = 15   # rows the sample misses
    values = (atoms[index] + 1e-3 * rng.standard_normal((vectors, group))).astype(np.float32)
    say("warm keep fit", group)
    host, dev = _both(vqdev, values.reshape(-1), group=group, init=atoms)
    np.testing.assert_array_equal(dev, host)
    np.testing.assert_array_equal(dev[15], atoms[15])


@pytest.mark.parametrize("group", [8, 16, 32])
@pytest.mark.parametrize("sample", [4096, 30000])
def test_identical_rows_reseed_every_empty_entry(vqdev, group, sample):
    """A book of identical rows sends the whole sample to entry 0 and empties
    the other fifteen, which are reseeded one after another: one 4,096-term
    in-order mean, then fifteen farthest-row searches. A 30,000-row sample
    takes several staging rounds and keeps the reseed gaps in memory."""
    rng = np.random.default_rng(100 + group)
    values = (rng.standard_normal(30000 * group) * 0.1).astype(np.float32)
    zero = np.zeros((16, group), np.float32)
    say("zero-book fit", group, sample)
    host, dev = _both(vqdev, values, group=group, init=zero, sample_vectors=sample)
    np.testing.assert_array_equal(dev, host)
    assert len(np.unique(dev, axis=0)) == 16


@pytest.mark.parametrize("group", [8, 16, 32])
@pytest.mark.parametrize("sample", [4096, 30000])
def test_books_with_copies_reseed_like_the_host_fit(vqdev, group, sample):
    """A warm book whose rows repeat (0 = 2 = 11, 1 = 6, 3 = 4 = 14, 7 = 8 = 9)
    and two distinct rows far from the data: the later copies and the far
    rows take no sample vector and are reseeded in turn. A reseed measures
    the book's untouched rows; a row with a copy at a higher index gives that
    copy's gap, so runs of reseeds separated only by copies share their
    distances, and the others measure afresh. The books must equal the host
    fit's, from a 4,096-row sample and from a 30,000-row one."""
    rng = np.random.default_rng(400 + group)
    atoms = rng.standard_normal((10, group)).astype(np.float32)
    rows = [0, 1, 0, 2, 2, 3, 1, 4, 4, 4, 5, 0, 6, 7, 2, 8]
    init = atoms[[r % 10 for r in rows]].copy()
    init[5] = 40.0                                 # far from every vector
    init[12] = -40.0
    pick = rng.integers(0, 10, 30000)
    values = (atoms[pick] + 0.3 * rng.standard_normal((30000, group))).astype(np.float32)
    say("fit with copied rows", group, sample)
    host, dev = _both(vqdev, values.reshape(-1), group=group, init=init, sample_vectors=sample)
    np.testing.assert_array_equal(dev, host)


@pytest.mark.parametrize("group,vectors", [(8, 3000), (8, 4096), (16, 2000)])
def test_lone_reseed_equals_the_host_fit(vqdev, group, vectors):
    """One entry of a warm book lies far from every vector, so the first
    iteration reseeds it alone, over a sample staged whole in LDS: the search
    that measures only the rows whose gap to their own entry reaches the best
    exact gap of 16 probe rows. Outlier rows (three identical, tying for the
    farthest gap) and a spread of distances must give the host fit's books."""
    rng = np.random.default_rng(500 + group + vectors)
    atoms = rng.standard_normal((15, group)).astype(np.float32)
    pick = rng.integers(0, 15, vectors)
    spread = rng.uniform(0.05, 0.6, (vectors, 1)).astype(np.float32)
    values = (atoms[pick] + spread * rng.standard_normal((vectors, group))).astype(np.float32)
    values[[700, 1500, 1900]] = 9.0
    init = np.concatenate([atoms, np.full((1, group), -30.0, np.float32)])
    say("lone reseed", group, vectors)
    host, dev = _both(vqdev, values.reshape(-1), group=group, init=init, sample_vectors=vectors)
    np.testing.assert_array_equal(dev, host)


@pytest.mark.parametrize("group", [8, 16])
def test_ties_and_collapses_equal_the_host_fit(vqdev, group):
    rng = np.random.default_rng(7)
    few = rng.integers(-2, 3, size=(6000, group)).astype(np.float32)   # many exact ties
    say("tie fit", group)
    host, dev = _both(vqdev, few.reshape(-1), group=group)
    np.testing.assert_array_equal(dev, host)
    same = np.full(500 * group, 0.25, np.float32)                      # one point only
    host, dev = _both(vqdev, same, group=group, init=rng.standard_normal((16, group)).astype(
        np.float32))
    np.testing.assert_array_equal(dev, host)


def test_device_fit_refusals(vqdev):
    from alelyon_compute_kit import ack
    with pytest.raises(ValueError, match="complete vector"):
        vqdev.fit_codebook(np.ones(7, np.float32), group=8)
    with pytest.raises(ValueError):
        vqdev.fit_codebook(np.ones(64, np.float32), group=12)
    with pytest.raises(ValueError):
        vqdev.fit_codebook(np.array([np.nan] * 16, np.float32), group=8)
    device = vqdev.device
    values = device.buffer(64 * 4)
    book = device.buffer(16 * 8 * 4)
    status = device.buffer(4)
    try:
        values.upload(np.full(64, np.inf, np.float32))
        status.upload(np.zeros(1, np.uint32))
        vqdev.fit_resident(values, 64, book, status, group=8)
        assert int(status.download(np.uint32)[0]) & 1
        with pytest.raises(ack.AckError):
            vqdev.fit_resident(values, 64, values, status, group=8)   # book aliases values
        with pytest.raises(ack.AckError):
            vqdev.fit_resident(values, 65, book, status, group=8)     # values too small
    finally:
        for b in (values, book, status):
            b.free()
